// Reader of the reference's `.viper` v1 artifact: the on-disk form of the
// quantized weights this path consumes (written by the reference's converter,
// tools/convert/convert.cpp:187-284; loaded by its engine,
// include/viper/model_impl.cuh:162-257).
//
// Layout (all integers little-endian):
//   16 bytes   magic "VIPER" + 11 zero bytes
//   40 bytes   u32 version (1), n_layers, n_passes, hidden, intermediate,
//              n_heads, n_kv_heads, head_dim, vocab, max_seq
//   sections   each a u64 byte count followed by that many bytes, in order:
//              for pass < n_passes, layer < n_layers: q, k, v, o, gate, up,
//                down, each as (packed Q4_G64, bf16 scales); every pass after
//                the first repeats the first (the reference skips them)
//              embed [vocab][hidden] bf16
//              lm_head (packed Q4_G64 [vocab][hidden], bf16 scales)
//              final norm [hidden] bf16
//              for pass, layer: input_layernorm, post_attention_layernorm,
//                each [hidden] bf16
//   Linear shapes (rows = outputs, cols = inputs): q (n_heads*head_dim,
//   hidden), k and v (n_kv_heads*head_dim, hidden), o (hidden,
//   n_heads*head_dim), gate and up (intermediate, hidden), down (hidden,
//   intermediate).
//
// Unlike the reference loader, parse() checks every section's size against
// the shape the header implies and rejects truncated or trailing data.
#pragma once

#include <array>
#include <string>
#include <vector>

#include "viper/common.h"
#include "viper/quant.h"
#include "viper/status.h"

namespace viper::artifact {

struct Header {
    u32 version = 0;
    u32 n_layers = 0;
    u32 n_passes = 0;
    u32 hidden = 0;
    u32 intermediate = 0;
    u32 n_heads = 0;
    u32 n_kv_heads = 0;
    u32 head_dim = 0;
    u32 vocab = 0;
    u32 max_seq = 0;
};

// A section's payload: byte offset in the file and byte count.
struct Blob {
    u64 offset = 0;
    u64 size = 0;
};

struct LinearBlob {
    Blob packed;
    Blob scales;
    i32 rows = 0;
    i32 cols = 0;
};

// Per-layer linears in file order.
enum Linear : int { Q = 0, K = 1, V = 2, O = 3, GATE = 4, UP = 5, DOWN = 6, N_LINEAR = 7 };

struct Index {
    Header header;
    std::vector<std::array<LinearBlob, N_LINEAR>> layers;  // first pass
    Blob embed;
    LinearBlob lm_head;
    Blob final_norm;
    std::vector<std::array<Blob, 2>> norms;  // {input_layernorm, post_attention_layernorm}, first pass
};

constexpr usize kHeaderBytes = 56;

// Validate and index an artifact held in memory.  INVALID_ARGUMENT (with the
// offending section named) for a bad magic, version, header or section size;
// IO_ERROR for truncated or trailing bytes.
Status parse(const u8* data, usize size, Index* out);

// A read-only memory map of a file.
class MappedFile {
  public:
    MappedFile() = default;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    ~MappedFile();
    Status open(const std::string& path);
    const u8* data() const noexcept { return data_; }
    usize size() const noexcept { return size_; }

  private:
    const u8* data_ = nullptr;
    usize size_ = 0;
};

// Device copy of an artifact's first pass: one device allocation holding
// every section at a 256-byte aligned offset (the kernels' alignment needs),
// and views into it.  Linears are Q4_G64 with bf16 scales.
struct DeviceModel {
    void* arena = nullptr;
    usize arena_bytes = 0;
    std::vector<std::array<quant::QuantizedWeight, N_LINEAR>> layers;
    quant::QuantizedWeight lm_head;
    void* embed = nullptr;       // [vocab][hidden] bf16
    void* final_norm = nullptr;  // [hidden] bf16
    std::vector<std::array<void*, 2>> norms;
};

// Allocate the arena and copy every section of `idx` from `data` (the bytes
// parse() indexed) to the device.  OUT_OF_MEMORY / CUDA_ERROR on device
// failures; `out` is left empty on failure.
Status upload(const u8* data, const Index& idx, DeviceModel* out);

// Free the arena (no-op for an empty model).
Status release(DeviceModel* model);

}  // namespace viper::artifact
