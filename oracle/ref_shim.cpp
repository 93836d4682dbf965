// Thin C-ABI wrappers around the reference's self-contained host decode helpers
// (orders/F1-ref/exl3_dequant.cuh:9-147), compiled from the header where it lies
// in the reference tree.  Test infrastructure only: used to cross-check the
// oracle's window extraction and to document where the reference CPU helper
// (truncating float->half) differs from the round-to-nearest canon.
#include EXL3_REF_HEADER

extern "C" {
uint16_t ref_read_window(const uint16_t* packed, size_t words, size_t bit) {
    return vllm_exl3::read_window(packed, words, bit);
}
uint16_t ref_decode_codebook_bits(uint16_t window, int cb) {
    return vllm_exl3::decode_codebook_bits(window, cb);
}
float ref_decode_weight(const uint16_t* packed, size_t words, int index, int bits, int mcg) {
    return vllm_exl3::decode_weight(packed, words, index, bits, mcg != 0);
}
float ref_half_bits_to_float(uint16_t h) { return vllm_exl3::half_bits_to_float(h); }
uint16_t ref_float_to_half_bits(float f) { return vllm_exl3::float_to_half_bits(f); }
void ref_hadamard(float* v, int n) { vllm_exl3::hadamard(v, n); }
}
