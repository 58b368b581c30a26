// Binds the reference converter's Q4_G64 weight quantizer so the oracle can
// be checked against the reference's own code.  TEST INFRASTRUCTURE ONLY.
//
// The reference file is compiled where it lies (its path comes from the
// Makefile as REF_CONVERT_CPP); only its main() is renamed so this shared
// library has no entry point of its own.  quantize_q4_g64 is file-static in
// the reference (tools/convert/convert.cpp:91-127), so it is reachable only
// from inside the same translation unit, which is why this wrapper includes
// the file instead of linking an object.
#include <cstdint>
#include <cstring>
#include <vector>

#define main viper_reference_convert_main
#include REF_CONVERT_CPP
#undef main

extern "C" int ref_quantize_q4_g64(const uint16_t* w_bf16, int N, int K, uint8_t* packed,
                                   uint16_t* scales_bf16) {
    if (!w_bf16 || !packed || !scales_bf16 || N <= 0 || K <= 0 || K % 64) return -1;
    std::vector<uint8_t> p;
    std::vector<uint16_t> s;
    quantize_q4_g64(w_bf16, N, K, p, s);
    std::memcpy(packed, p.data(), p.size());
    std::memcpy(scales_bf16, s.data(), s.size() * sizeof(uint16_t));
    return 0;
}
