// Test-side writer of a synthetic `.viper` v1 artifact (the layout of
// include/viper/artifact.h, as the reference converter writes it,
// tools/convert/convert.cpp:187-284): small dimensions, every section filled
// by a caller-supplied function, later passes repeating the first.
#pragma once

#include <cstdint>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

struct ArtifactDims {
    uint32_t layers = 2, passes = 2, hidden = 128, inter = 256, heads = 2, kv_heads = 1, head_dim = 64,
             vocab = 300, max_seq = 4096;
};

// fill(name, layer, bytes, out): bytes of one section; name is "q_proj",
// ..., "down_proj" (+ ".scales" for the scale half), "embed", "lm_head",
// "lm_head.scales", "final_norm", "input_layernorm", "post_attention_layernorm".
using SectionFill = std::function<void(const std::string& name, int layer, size_t bytes, std::vector<uint8_t>& out)>;

inline std::vector<uint8_t> write_artifact(const ArtifactDims& d, const SectionFill& fill, uint32_t version = 1) {
    std::vector<uint8_t> f;
    auto put = [&](const void* p, size_t n) { f.insert(f.end(), (const uint8_t*)p, (const uint8_t*)p + n); };
    const char magic[16] = {'V', 'I', 'P', 'E', 'R'};
    put(magic, 16);
    const uint32_t hdr[10] = {version, d.layers, d.passes, d.hidden, d.inter, d.heads, d.kv_heads, d.head_dim,
                              d.vocab, d.max_seq};
    put(hdr, sizeof(hdr));
    auto section = [&](const std::string& name, int layer, size_t bytes) {
        std::vector<uint8_t> b;
        fill(name, layer, bytes, b);
        const uint64_t n = b.size();
        put(&n, 8);
        put(b.data(), b.size());
    };
    const size_t H = d.hidden, I = d.inter, nQ = (size_t)d.heads * d.head_dim, nKV = (size_t)d.kv_heads * d.head_dim;
    const char* names[7] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};
    const size_t rows[7] = {nQ, nKV, nKV, H, I, I, H};
    const size_t cols[7] = {H, H, H, nQ, H, H, I};
    for (uint32_t p = 0; p < d.passes; ++p)
        for (uint32_t l = 0; l < d.layers; ++l)
            for (int i = 0; i < 7; ++i) {
                section(names[i], (int)l, rows[i] * cols[i] / 2);
                section(std::string(names[i]) + ".scales", (int)l, rows[i] * (cols[i] / 64) * 2);
            }
    section("embed", -1, (size_t)d.vocab * H * 2);
    section("lm_head", -1, (size_t)d.vocab * H / 2);
    section("lm_head.scales", -1, (size_t)d.vocab * (H / 64) * 2);
    section("final_norm", -1, H * 2);
    for (uint32_t p = 0; p < d.passes; ++p)
        for (uint32_t l = 0; l < d.layers; ++l) {
            section("input_layernorm", (int)l, H * 2);
            section("post_attention_layernorm", (int)l, H * 2);
        }
    return f;
}

// Deterministic filler: bytes from a hash of (name, layer, position).
inline void hash_fill(const std::string& name, int layer, size_t bytes, std::vector<uint8_t>& out) {
    uint64_t h = 1469598103934665603ull;
    for (char c : name) h = (h ^ (uint8_t)c) * 1099511628211ull;
    h ^= (uint64_t)(layer + 7) * 0x9e3779b97f4a7c15ull;
    out.resize(bytes);
    for (size_t i = 0; i < bytes; ++i) {
        uint64_t z = h + i * 0x9e3779b97f4a7c15ull;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        out[i] = (uint8_t)(z ^ (z >> 31));
    }
}
