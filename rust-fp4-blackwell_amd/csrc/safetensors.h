// Read-only safetensors file: 8-byte little-endian header length, a JSON
// header {name: {"dtype", "shape", "data_offsets"}, "__metadata__": {...}},
// then the tensor bytes.  The file is memory-mapped; tensors are views.
// The reference reads the same format (llama_run/src/main.rs:413-430).
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace rfp4 {

struct StTensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0; // byte offsets into the data section
    uint64_t numel() const
    {
        uint64_t n = 1;
        for (uint64_t d : shape) n *= d;
        return n;
    }
};

class StFile {
  public:
    ~StFile();
    // Opens and validates path; on failure returns an RFP4_E_* code with the
    // library's error text set.
    int open(const char *path);
    const StTensor *find(const std::string &name) const;
    const std::vector<StTensor> &tensors() const { return tensors_; }
    const uint8_t *data(const StTensor &t) const { return data_ + t.begin; }
    // Element size of a dtype name, 0 if unknown.
    static uint32_t dtype_bytes(const std::string &dtype);
    // The tensor widened to f32 (BF16, F16, F32), exactly as the reference's
    // `get` closure (llama_run/src/main.rs:419-430).
    int read_f32(const StTensor &t, float *out, uint64_t count) const;
    // The tensor as fp16 bits: F16 as stored, BF16 / F32 rounded to nearest
    // even (exact for bf16 values of magnitude 2^-17 .. 65504).
    int read_f16(const StTensor &t, uint16_t *out, uint64_t count) const;

  private:
    int fd_ = -1;
    uint8_t *map_ = nullptr;
    size_t map_len_ = 0;
    const uint8_t *data_ = nullptr;
    uint64_t data_len_ = 0;
    std::vector<StTensor> tensors_;
};

// Host conversions shared by the loaders (exact where the target holds the value).
float f16_to_f32_host(uint16_t h);
uint16_t f32_to_bf16_rne_host(float f);
uint16_t f32_to_f16_rne_host(float f); // IEEE binary16, round to nearest even, overflow to inf

} // namespace rfp4
