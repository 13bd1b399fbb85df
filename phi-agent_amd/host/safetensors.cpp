// Safetensors reading and the quantized-weight layout rules; see safetensors.hpp.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "phi_media.hpp"

namespace phi::media {

// ---------------------------------------------------------------- JSON
// A small recursive-descent reader for the two JSON documents involved (the
// safetensors header and the comfy_quant blob): objects, arrays, strings with
// the standard escapes, numbers, true / false / null.
namespace {

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    int64_t inum = 0;  // exact value of an integral number
    bool integral = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
public:
    JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(Json& out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

private:
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t c) {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xc0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3f));
        } else if (c < 0x10000) {
            s += (char)(0xe0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3f));
            s += (char)(0x80 | (c & 0x3f));
        } else {
            s += (char)(0xf0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3f));
            s += (char)(0x80 | ((c >> 6) & 0x3f));
            s += (char)(0x80 | (c & 0x3f));
        }
    }
    bool hex4(uint32_t& v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t v;
                    if (!hex4(v)) return false;
                    if (v >= 0xd800 && v < 0xdc00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        uint32_t lo;
                        if (!hex4(lo) || lo < 0xdc00 || lo >= 0xe000) return false;
                        v = 0x10000 + ((v - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(s, v);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        p_++;
        return true;
    }
    bool number(Json& j) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') p_++;
        bool frac = false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                             *p_ == '-')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
            p_++;
        }
        if (p_ == s) return false;
        const std::string t(s, p_);
        char* e = nullptr;
        j.kind = Json::Num;
        j.num = strtod(t.c_str(), &e);
        if (!e || *e) return false;
        if (!frac) {
            errno = 0;
            j.inum = strtoll(t.c_str(), &e, 10);
            j.integral = errno == 0 && e && !*e;
        }
        return true;
    }
    bool value(Json& j, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            p_++;
            j.kind = Json::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                p_++;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_++ != ':') return false;
                Json v;
                if (!value(v, depth + 1)) return false;
                j.obj.emplace_back(std::move(key), std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            p_++;
            j.kind = Json::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                p_++;
                return true;
            }
            for (;;) {
                Json v;
                if (!value(v, depth + 1)) return false;
                j.arr.push_back(std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            j.kind = Json::Str;
            return string(j.str);
        }
        if (lit("true")) {
            j.kind = Json::Bool;
            j.b = true;
            return true;
        }
        if (lit("false")) {
            j.kind = Json::Bool;
            return true;
        }
        if (lit("null")) return true;
        return number(j);
    }
};

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

std::string weight_stem(const std::string& name) { return ends_with(name, ".weight") ? name.substr(0, name.size() - 7) : name; }

// The dtype spellings a header may use: the safetensors names plus the torch
// and short spellings the reference's reader accepts (dtype_from_name,
// core/util/media_common.cpp:31-44).  I4 / U4 / int4 hold two values per byte;
// their shape keeps the packed width.  Anything else is unknown, and such an
// entry is skipped as the reference skips it (core/host/st.cpp:242).
StDType dtype_of(const std::string& s) {
    static const std::pair<const char*, StDType> table[] = {
        {"F32", StDType::F32},         {"float32", StDType::F32},      {"float", StDType::F32},
        {"F16", StDType::F16},         {"float16", StDType::F16},      {"BF16", StDType::BF16},
        {"bfloat16", StDType::BF16},   {"I8", StDType::I8},            {"int8", StDType::I8},
        {"U8", StDType::U8},           {"uint8", StDType::U8},         {"I4", StDType::I4},
        {"int4", StDType::I4},         {"U4", StDType::I4},            {"F8_E4M3", StDType::F8_E4M3},
        {"float8_e4m3fn", StDType::F8_E4M3}, {"float8_e4m3", StDType::F8_E4M3}, {"F8E4M3", StDType::F8_E4M3},
        {"e4m3", StDType::F8_E4M3},    {"F8_E5M2", StDType::F8_E5M2},  {"float8_e5m2", StDType::F8_E5M2},
        {"F8E5M2", StDType::F8_E5M2},  {"e5m2", StDType::F8_E5M2},     {"F64", StDType::F64},
        {"I64", StDType::I64},         {"I32", StDType::I32},          {"I16", StDType::I16},
        {"BOOL", StDType::BOOL}};
    for (const auto& e : table)
        if (s == e.first) return e.second;
    return StDType::Unknown;
}

float half_bits_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {  // subnormal: m * 2^-24, exact in fp32
            float f = std::ldexp((float)m, -24);
            std::memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float f8_to_f32(uint8_t b, bool e4m3) {
    const bool neg = b & 0x80;
    float v;
    if (e4m3) {
        const int e = (b >> 3) & 15, m = b & 7;
        if (e == 15 && m == 7) return NAN;
        v = e == 0 ? std::ldexp((float)m, -9) : std::ldexp((float)(8 + m), e - 10);
    } else {
        const int e = (b >> 2) & 31, m = b & 3;
        if (e == 31) return m == 0 ? (neg ? -INFINITY : INFINITY) : NAN;
        v = e == 0 ? std::ldexp((float)m, -16) : std::ldexp((float)(4 + m), e - 17);
    }
    return neg ? -v : v;
}

}  // namespace

const char* st_dtype_name(StDType t) {
    switch (t) {
        case StDType::F64: return "F64";
        case StDType::F32: return "F32";
        case StDType::F16: return "F16";
        case StDType::BF16: return "BF16";
        case StDType::I64: return "I64";
        case StDType::I32: return "I32";
        case StDType::I16: return "I16";
        case StDType::I8: return "I8";
        case StDType::U8: return "U8";
        case StDType::BOOL: return "BOOL";
        case StDType::F8_E4M3: return "F8_E4M3";
        case StDType::F8_E5M2: return "F8_E5M2";
        case StDType::I4: return "I4";
        default: return "?";
    }
}

size_t st_dtype_bytes(StDType t) {
    switch (t) {
        case StDType::F64:
        case StDType::I64: return 8;
        case StDType::F32:
        case StDType::I32: return 4;
        case StDType::F16:
        case StDType::BF16:
        case StDType::I16: return 2;
        case StDType::I8:
        case StDType::U8:
        case StDType::I4:  // packed: two values per byte, the shape holds bytes
        case StDType::BOOL:
        case StDType::F8_E4M3:
        case StDType::F8_E5M2: return 1;
        default: return 0;
    }
}

// ---------------------------------------------------------------- comfy_quant

QuantSpec parse_quant_spec(const void* json_bytes, size_t len) {
    QuantSpec spec;
    if (!json_bytes || len == 0) return spec;
    std::string text((const char*)json_bytes, len);
    const size_t end = text.find_last_of('}');
    if (end == std::string::npos) return spec;
    text.resize(end + 1);
    Json j;
    if (!JsonReader(text.data(), text.size()).parse(j) || j.kind != Json::Obj) return spec;
    const Json* f = j.get("format");
    spec.format = f && f->kind == Json::Str ? f->str : "int8_tensorwise";
    const Json* c = j.get("convrot");
    spec.convrot = c && c->kind == Json::Bool && c->b;
    const Json* g = j.get("convrot_groupsize");
    spec.convrot_groupsize = g && g->kind == Json::Num ? (int)g->num : 256;
    if (spec.convrot_groupsize <= 0) spec.convrot_groupsize = 256;
    const Json* gs = j.get("group_size");
    spec.group_size = gs && gs->kind == Json::Num ? (int)gs->num : 0;
    if (spec.group_size < 0) spec.group_size = 0;
    spec.valid = true;
    return spec;
}

bool parse_number_records(const std::string& text, const std::string& key,
                          std::vector<std::map<std::string, double>>* out) {
    Json doc;
    if (!JsonReader(text.data(), text.size()).parse(doc) || doc.kind != Json::Obj) return false;
    const Json* arr = doc.get(key);
    if (!arr || arr->kind != Json::Arr) return false;
    out->clear();
    for (const Json& rec : arr->arr) {
        if (rec.kind != Json::Obj) return false;
        std::map<std::string, double> m;
        for (const auto& kv : rec.obj)
            if (kv.second.kind == Json::Num) m[kv.first] = kv.second.num;
        out->push_back(std::move(m));
    }
    return true;
}

int quant_bits_per_weight(const std::string& format) {
    if (format == "asym_w4a8_int8" || format == "nvfp4" || format == "mxfp4") return 4;
    if (format == "w6a8_int8" || format == "w6a8") return 6;
    return 8;
}

// ---------------------------------------------------------------- file

SafeTensors::SafeTensors(const std::string& path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw MediaError("safetensors: cannot open " + path);
    struct stat sb;
    if (fstat(fd_, &sb) != 0 || sb.st_size < 8) {
        ::close(fd_);
        throw MediaError("safetensors: " + path + " is too short");
    }
    map_bytes_ = (size_t)sb.st_size;
    map_ = mmap(nullptr, map_bytes_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) {
        ::close(fd_);
        throw MediaError("safetensors: cannot map " + path);
    }
    auto fail = [&](const std::string& why) {
        munmap(map_, map_bytes_);
        ::close(fd_);
        throw MediaError("safetensors: " + path + ": " + why);
    };
    const uint8_t* base = (const uint8_t*)map_;
    uint64_t hlen = 0;
    for (int i = 0; i < 8; i++) hlen |= (uint64_t)base[i] << (8 * i);
    if (hlen > map_bytes_ - 8) fail("header length " + std::to_string(hlen) + " runs past the file");
    Json h;
    if (!JsonReader((const char*)base + 8, (size_t)hlen).parse(h) || h.kind != Json::Obj) fail("malformed header");
    const uint64_t data0 = 8 + hlen, data_bytes = map_bytes_ - data0;
    for (const auto& kv : h.obj) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind == Json::Obj)
                for (const auto& m : kv.second.obj)
                    if (m.second.kind == Json::Str) metadata_[m.first] = m.second.str;
            continue;
        }
        const Json& e = kv.second;
        // As the reference reads a header (core/host/st.cpp:231-271): entries that
        // are not objects, whose dtype it cannot name or that have no two-element
        // data_offsets are skipped; a malformed shape or offsets past the data
        // are errors.
        if (e.kind != Json::Obj) continue;
        const Json* dt = e.get("dtype");
        const Json* sh = e.get("shape");
        const Json* off = e.get("data_offsets");
        if (!dt || dt->kind != Json::Str) continue;
        StTensor t;
        t.name = kv.first;
        t.dtype = dtype_of(dt->str);
        if (t.dtype == StDType::Unknown) continue;
        if (!off || off->kind != Json::Arr || off->arr.size() != 2) continue;
        if (!sh || sh->kind != Json::Arr) fail("entry '" + kv.first + "' has no shape");
        t.numel = 1;
        for (const Json& d : sh->arr) {
            if (d.kind != Json::Num || !d.integral || d.inum < 0) fail("entry '" + kv.first + "' has a bad shape");
            t.shape.push_back(d.inum);
            if (__builtin_mul_overflow(t.numel, d.inum, &t.numel))
                fail("entry '" + kv.first + "' has a shape whose element count overflows");
        }
        if (!off->arr[0].integral || !off->arr[1].integral) fail("entry '" + kv.first + "' has bad offsets");
        const int64_t b = off->arr[0].inum, en = off->arr[1].inum;
        if (b < 0 || en < b || (uint64_t)en > data_bytes) fail("entry '" + kv.first + "' lies outside the file");
        t.offset = data0 + (uint64_t)b;
        t.nbytes = (uint64_t)(en - b);
        uint64_t want = 0;
        if (__builtin_mul_overflow((uint64_t)t.numel, (uint64_t)st_dtype_bytes(t.dtype), &want) || want != t.nbytes)
            fail("entry '" + kv.first + "' has " + std::to_string(t.nbytes) + " bytes for " +
                 std::to_string(t.numel) + " " + st_dtype_name(t.dtype) + " values");
        t.data = base + t.offset;
        if (!tensors_.count(t.name)) order_.push_back(t.name);
        tensors_[t.name] = std::move(t);
    }
    if (tensors_.empty()) fail("no readable tensors");
}

SafeTensors::~SafeTensors() {
    if (map_ && map_ != MAP_FAILED) munmap(map_, map_bytes_);
    if (fd_ >= 0) ::close(fd_);
}

const StTensor* SafeTensors::find(const std::string& name) const {
    const auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

const StTensor& SafeTensors::require(const std::string& name) const {
    const StTensor* t = find(name);
    if (!t) throw MediaError("tensor not found: " + name);
    return *t;
}

QuantSpec SafeTensors::quant_spec_of(const std::string& weight_name) const {
    std::vector<std::string> cands;
    if (ends_with(weight_name, ".weight")) cands.push_back(weight_name.substr(0, weight_name.size() - 7) + ".comfy_quant");
    if (ends_with(weight_name, ".weight_scale"))
        cands.push_back(weight_name.substr(0, weight_name.size() - 13) + ".comfy_quant");
    cands.push_back(weight_name + ".comfy_quant");
    for (const auto& c : cands)
        if (const StTensor* q = find(c)) return parse_quant_spec(q->data, (size_t)q->nbytes);
    return QuantSpec{};
}

SafeTensors::WeightLayout SafeTensors::weight_layout(const std::string& weight_name) const {
    WeightLayout L;
    const std::string base = weight_stem(weight_name);
    L.spec = quant_spec_of(weight_name);
    L.codebook = find(base + ".weight_codebook");
    L.rel_scale = find(base + ".weight_s_rel");
    L.correction = find(base + ".weight_correction");
    L.row_scale = find(base + ".weight_s_channel");
    if (!L.row_scale) L.row_scale = find(base + ".weight_scale");
    L.global_scale = find(base + ".weight_scale_2");
    const std::string& f = L.spec.format;
    if (f == "nvfp4" || f == "mxfp4") {
        // Two scales, told apart by shape (core/host/st.cpp:850-880): the block
        // table holds one entry per block (>= 2-D, more than one value), the
        // global scale one value.  ComfyUI writes the table as weight_scale and
        // the global as weight_scale_2; a file with the names swapped is read
        // the same way.  fp4 has no per-row scale.
        const auto table = [](const StTensor* t) { return t && t->numel > 1 && t->shape.size() >= 2; };
        if (!L.rel_scale && table(L.row_scale)) {
            L.rel_scale = L.row_scale;
            L.row_scale = nullptr;
        } else if (table(L.global_scale) && !table(L.rel_scale)) {
            L.rel_scale = L.global_scale;
            L.global_scale = L.row_scale;
            L.row_scale = nullptr;
        }
    }
    L.bits = quant_bits_per_weight(L.spec.format);
    if (f == "asym_w4a8_int8" || f == "w6a8_int8" || f == "w6a8") {
        // Both grouped families store a convrot-rotated weight (the blob carries
        // convrot_groupsize rather than a convrot flag).
        L.packed = true;
        L.group = L.spec.group_size > 0 ? L.spec.group_size : (f == "asym_w4a8_int8" ? 16 : 32);
        L.known_family = true;
        L.spec.convrot = true;
        if (L.spec.convrot_groupsize <= 0) L.spec.convrot_groupsize = 256;
    } else if (f == "int8_tensorwise" || f == "int8") {
        L.group = L.rel_scale ? (L.spec.group_size > 0 ? L.spec.group_size : 32) : 0;
        L.known_family = true;
    } else if (f == "convrot_w4a4") {
        L.spec.convrot = true;
        if (L.spec.convrot_groupsize <= 0) L.spec.convrot_groupsize = 256;
        L.known_family = true;
    } else if (f == "nvfp4" || f == "mxfp4") {
        L.packed = true;
        L.group = L.spec.group_size > 0 ? L.spec.group_size : 16;
        L.known_family = true;
    } else if (f == "fp8" || f == "float8_e4m3fn" || f == "float8_e4m3" || f == "float8_e5m2") {
        L.known_family = true;
    }
    return L;
}

int64_t SafeTensors::logical_cols(const StTensor& t) const {
    if (t.shape.empty()) return 0;
    const int64_t stored = t.shape.back();
    const WeightLayout L = weight_layout(t.name);
    if (L.packed && L.bits > 0) return stored * 8 / L.bits;
    if (L.spec.valid && L.spec.format == "convrot_w4a4") return stored * 2;
    // A bare packed int4 (I4 / U4 with no sidecar): two values per byte along K.
    if (t.dtype == StDType::I4) return stored * 2;
    return stored;
}

bool SafeTensors::is_plain_int8(const StTensor& t) const {
    if (t.dtype != StDType::I8) return false;
    const WeightLayout L = weight_layout(t.name);
    if (L.packed || L.rel_scale) return false;
    if (L.spec.valid && !L.spec.format.empty() && L.spec.format != "int8_tensorwise") return false;
    return find(weight_stem(t.name) + ".weight_scale") != nullptr;
}

std::vector<float> SafeTensors::to_f32(const StTensor& t) const {
    std::vector<float> v((size_t)t.numel);
    for (int64_t i = 0; i < t.numel; i++) {
        switch (t.dtype) {
            case StDType::F32: std::memcpy(&v[(size_t)i], t.data + 4 * i, 4); break;
            case StDType::F16: {
                uint16_t h;
                std::memcpy(&h, t.data + 2 * i, 2);
                v[(size_t)i] = half_bits_to_f32(h);
                break;
            }
            case StDType::BF16: {
                uint16_t h;
                std::memcpy(&h, t.data + 2 * i, 2);
                const uint32_t u = (uint32_t)h << 16;
                std::memcpy(&v[(size_t)i], &u, 4);
                break;
            }
            case StDType::F8_E4M3: v[(size_t)i] = f8_to_f32(t.data[i], true); break;
            case StDType::F8_E5M2: v[(size_t)i] = f8_to_f32(t.data[i], false); break;
            default: throw MediaError("'" + t.name + "': " + st_dtype_name(t.dtype) + " is not a float tensor");
        }
    }
    return v;
}

float SafeTensors::row_scale_value(const StTensor& scale, int64_t row) const {
    if (scale.numel == 0) return 1.0f;
    const int64_t i = scale.numel == 1 ? 0 : row;
    if (i < 0 || i >= scale.numel)
        throw MediaError("'" + scale.name + "' has " + std::to_string(scale.numel) + " scales but row " +
                         std::to_string(row) + " was asked for");
    switch (scale.dtype) {
        case StDType::F32: {
            float v;
            std::memcpy(&v, scale.data + 4 * i, 4);
            return v;
        }
        case StDType::F16: {
            uint16_t h;
            std::memcpy(&h, scale.data + 2 * i, 2);
            return half_bits_to_f32(h);
        }
        case StDType::BF16: {
            uint16_t h;
            std::memcpy(&h, scale.data + 2 * i, 2);
            const uint32_t u = (uint32_t)h << 16;
            float v;
            std::memcpy(&v, &u, 4);
            return v;
        }
        case StDType::F8_E4M3:
        case StDType::U8: return f8_to_f32(scale.data[i], true);
        case StDType::F8_E5M2: return f8_to_f32(scale.data[i], false);
        default: throw MediaError("'" + scale.name + "': scale dtype " + st_dtype_name(scale.dtype) + " is not readable");
    }
}

}  // namespace phi::media
