"""Writers of small safetensors checkpoints in the layouts the C++ host layer
reads (int8_tensorwise, asym_w4a8_int8, w6a8_int8, convrot_w4a4), and a runner
for tests/cpp/st_tool.  Test infrastructure."""
import json
import os
import subprocess

import numpy as np
import torch
from safetensors.torch import save_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ST_TOOL = os.path.join(ROOT, "tests", "cpp", "st_tool")


def comfy_blob(spec: dict, width: int = 72) -> torch.Tensor:
    """The comfy_quant sidecar: UTF-8 JSON, zero-padded to a fixed width."""
    b = json.dumps(spec).encode()
    b = b.ljust(max(width, len(b)), b"\0")
    return torch.frombuffer(bytearray(b), dtype=torch.uint8).clone()


def write(path: str, tensors: dict) -> str:
    save_file({k: v.contiguous() for k, v in tensors.items()}, path)
    return path


def run(*args, check=True):
    out = subprocess.run([ST_TOOL, *[str(a) for a in args]], capture_output=True, text=True, timeout=120)
    if check and out.returncode != 0:
        raise AssertionError(f"st_tool {args[0]} failed ({out.returncode}): {out.stdout} {out.stderr}")
    return out


def probe(path: str, base: str) -> dict:
    return json.loads(run("probe", path, base).stdout)


def write_raw(path: str, entries, metadata=None) -> str:
    """A safetensors file written by hand, so the header can use any dtype
    spelling, shape or offsets.  entries: (name, dtype string, shape,
    payload bytes or None for a header-only entry, extra header fields)."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for e in entries:
        name, dt, shape, payload = e[:4]
        extra = e[4] if len(e) > 4 else {}
        ent = {"dtype": dt, "shape": list(shape)}
        if payload is not None:
            ent["data_offsets"] = [off, off + len(payload)]
            blobs.append(payload)
            off += len(payload)
        ent.update(extra)
        header[name] = ent
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)
    return path


def lora_file(path: str, tensors: dict, metadata=None) -> str:
    """A LoRA factor file (safetensors, optional string metadata)."""
    save_file({k: v.contiguous() for k, v in tensors.items()}, path, metadata=metadata)
    return path
