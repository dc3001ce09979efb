// oracle/ref_shim.cpp -- C entry points over the reference's own dequant code.
//
// TEST INFRASTRUCTURE.  Compiled together with the reference's unmodified
// src/loader/dequant.cpp and src/loader/gguf.cpp (read in place under
// /root/reference, never copied) into oracle/_ref/libknj_ref.so, so the tests can
// check this repo's oracle against the functions Kanjoos actually runs:
//   fp16_to_fp32 / bf16_to_fp32   dequant.cpp:1032-1073
//   dequant_row_f32               dequant.cpp:1114-1256
//   dequant_dot_f32               dequant.cpp:1075-1112
#include <cstdint>

#include "src/loader/dequant.h"

extern "C" {

float knjr_fp16_to_fp32(uint16_t h) { return knj::fp16_to_fp32(h); }
float knjr_bf16_to_fp32(uint16_t b) { return knj::bf16_to_fp32(b); }

void knjr_dequant_row_f32(int type, const uint8_t* src, float* dst, uint64_t n) {
  knj::dequant_row_f32(static_cast<knj::GgmlType>(type), src, dst, n);
}

float knjr_dequant_dot_f32(int type, const uint8_t* src, const float* x, uint64_t n) {
  return knj::dequant_dot_f32(static_cast<knj::GgmlType>(type), src, x, n);
}

}  // extern "C"
