// Checkpoint reading for the quantized linear: safetensors files, the
// `comfy_quant` sidecar and the weight-layout rules of the families the
// library runs (core/host/st.hpp:218-253, core/host/st.cpp:811-935,
// core/host/quant.hpp:24-50, core/host/quant.cpp:18-52).
//
//   int8_tensorwise  <base>.weight I8 [N, K], <base>.weight_scale F32 [N]
//   asym_w4a8_int8   <base>.weight I8/U8 [N, K/2] nibbles (low first),
//                    <base>.weight_s_rel [N, K/group], <base>.weight_s_channel
//                    (or .weight_scale) F32 [N] or [1], optional
//                    <base>.weight_codebook F32 [16], <base>.weight_correction
//   w6a8_int8        as above with [N, K/2 + K/4] six-bit codes, no codebook
//   convrot_w4a4     <base>.weight I8 [N, K/2] signed nibbles, .weight_scale F32 [N]
//   nvfp4 / mxfp4    <base>.weight U8/I8 [N, K/2] E2M1 nibbles (even column in the
//                    HIGH nibble), a per-block scale table in the cuBLAS tiled
//                    layout (fp8, as .weight_scale or .weight_scale_2) and one
//                    global scale (the other of the two)
//   fp8              <base>.weight F8_E4M3 / F8_E5M2 [N, K], optional
//                    .weight_scale [N] or [1]
//   <base>.comfy_quant  U8 tensor holding a padded UTF-8 JSON blob
//
// The file is mapped read-only; tensors are views into the mapping.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace phi::media {

// I4 is a packed dtype: two signed nibbles per byte, the shape holds the bytes.
enum class StDType { Unknown, F64, F32, F16, BF16, I64, I32, I16, I8, U8, BOOL, F8_E4M3, F8_E5M2, I4 };

const char* st_dtype_name(StDType t);
size_t st_dtype_bytes(StDType t);

struct StTensor {
    std::string name;
    StDType dtype = StDType::Unknown;
    std::vector<int64_t> shape;
    int64_t numel = 0;
    uint64_t offset = 0;  // byte offset of the data within the file
    uint64_t nbytes = 0;
    const uint8_t* data = nullptr;  // into the mapping
    // Bytes of one stored row (the last dimension), as laid out on disk.
    uint64_t row_bytes() const {
        return shape.empty() ? nbytes : (uint64_t)shape.back() * st_dtype_bytes(dtype);
    }
};

// Parsed `comfy_quant` blob (core/host/quant.hpp:24-50).
struct QuantSpec {
    std::string format;  // "int8_tensorwise" | "asym_w4a8_int8" | "w6a8_int8" | "convrot_w4a4" | ...
    bool convrot = false;
    int convrot_groupsize = 256;
    int group_size = 0;
    bool valid = false;
};

// The blob is a fixed-size padded buffer: the text is cut at its last '}'.
// An unparsable blob yields an invalid spec (core/host/quant.cpp:18-38).
QuantSpec parse_quant_spec(const void* json_bytes, size_t len);

// Bits per weight on disk for a family (core/host/quant.cpp:40-52).
int quant_bits_per_weight(const std::string& format);

// The objects of a top-level array `key` in a JSON document, each as its
// numeric members (other members are left out).  False when the text does not
// parse or has no such array.
bool parse_number_records(const std::string& text, const std::string& key,
                          std::vector<std::map<std::string, double>>* out);

class SafeTensors {
public:
    // Maps the file and parses its header; throws MediaError on a malformed file.
    explicit SafeTensors(const std::string& path);
    ~SafeTensors();
    SafeTensors(const SafeTensors&) = delete;
    SafeTensors& operator=(const SafeTensors&) = delete;

    const StTensor* find(const std::string& name) const;
    const StTensor& require(const std::string& name) const;
    const std::map<std::string, StTensor>& tensors() const { return tensors_; }
    const std::string& path() const { return path_; }
    // Names of the readable entries in header order, and the header's
    // __metadata__ strings (core/host/st.cpp:231-241).
    const std::vector<std::string>& names() const { return order_; }
    const std::map<std::string, std::string>& metadata() const { return metadata_; }
    // Every value of a float tensor (F32 / F16 / BF16 / F8) as fp32, exactly.
    std::vector<float> to_f32(const StTensor& t) const;

    // The comfy_quant spec of a weight ("<base>.weight" -> "<base>.comfy_quant").
    QuantSpec quant_spec_of(const std::string& weight_name) const;

    // What a weight is on disk (core/host/st.hpp:223-237, st.cpp:839-925).
    struct WeightLayout {
        QuantSpec spec;
        int bits = 8;
        int64_t group = 0;
        const StTensor* row_scale = nullptr;   // weight_s_channel, else weight_scale
        const StTensor* rel_scale = nullptr;   // weight_s_rel
        const StTensor* codebook = nullptr;    // weight_codebook
        const StTensor* correction = nullptr;  // weight_correction
        const StTensor* global_scale = nullptr;  // nvfp4 / mxfp4: the one per-tensor scale
        bool packed = false;                   // bits < 8: the last dim is not K
        bool known_family = false;
    };
    WeightLayout weight_layout(const std::string& weight_name) const;

    // Logical K of a weight: stored bytes * 8 / bits for a packed family, twice the
    // stored width for convrot_w4a4, the last dimension otherwise.
    int64_t logical_cols(const StTensor& t) const;

    // The original int8 tensorwise form: I8 codes, one scale per row, no group table.
    bool is_plain_int8(const StTensor& t) const;

    // One value of a scale table for one row (a one-entry table broadcasts).
    float row_scale_value(const StTensor& scale, int64_t row) const;

private:
    std::string path_;
    int fd_ = -1;
    void* map_ = nullptr;
    size_t map_bytes_ = 0;
    std::map<std::string, StTensor> tensors_;
    std::vector<std::string> order_;
    std::map<std::string, std::string> metadata_;
};

}  // namespace phi::media
