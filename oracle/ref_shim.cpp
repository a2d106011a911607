// Thin C-ABI driver over the reference's own host decode header, compiled
// from the file where it lies under /root/reference (nothing is copied).
// Used only to validate the C restatement in exl3_oracle.c and to write the
// golden vectors under tests/golden/.  TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <cstddef>
#include EXL3_REF_HEADER

using namespace sglang_exl3;

extern "C" {
uint16_t ref_read_window(const uint16_t* packed, size_t words, size_t bit) {
    return read_window(packed, words, bit);
}
uint16_t ref_decode_codebook_bits(uint16_t window, int cb) { return decode_codebook_bits(window, cb); }
uint16_t ref_float_to_half_bits(float v) { return float_to_half_bits(v); }
float ref_half_bits_to_float(uint16_t h) { return half_bits_to_float(h); }
uint32_t ref_lop3_6a(uint32_t a, uint32_t b, uint32_t c) { return lop3_6a(a, b, c); }
void ref_hadamard(float* v, int n) { hadamard(v, n); }
float ref_decode_weight(const uint16_t* packed, size_t words, int index, int bits, int mcg) {
    return decode_weight(packed, words, index, bits, mcg != 0);
}
float ref_decode_mcg(uint16_t w) { return decode_mcg(w); }
float ref_decode_mul1(uint16_t w) { return decode_mul1(w); }
}
