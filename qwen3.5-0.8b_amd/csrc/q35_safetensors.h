// safetensors container parsing (host code): an 8-byte little-endian header length, a JSON
// header {name: {"dtype", "shape", "data_offsets": [begin, end)}, "__metadata__": {...}}, then
// the raw tensor bytes (offsets relative to the end of the header).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace q35 {

struct StTensor {
    std::string name;
    std::string dtype;            // "BF16", "F16", "F32", ...
    std::vector<int64_t> shape;
    const uint8_t* data = nullptr;
    size_t bytes = 0;
};

// Parses and validates the container (header bounds, JSON, dtype sizes, offsets inside the
// data region and equal to numel x element size). Returns false with `err` set on failure.
bool parse_safetensors(const void* file, size_t n, std::vector<StTensor>& out, std::string& err);

// bf16 bits of a tensor stored as BF16, F16 or F32: F32 (and F16 via its exact f32 value)
// is rounded to nearest even, as torch's Tensor.to(torch.bfloat16); NaN stays a quiet NaN.
bool to_bf16(const StTensor& t, std::vector<uint16_t>& out, std::string& err);

}  // namespace q35
