// Launchers of the gfx950 kernels (internal to the library; the C ABI wraps them).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "layout.hpp"

namespace syn {

// act_quant.hip
void launch_act_quant(int kind, const float* x, uint64_t rows, uint64_t k, uint8_t* ws,
                      hipStream_t stream);
// gemv.hip
void launch_gemv_q(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int rows,
                   float* y, hipStream_t stream);
// gemv_q4k.hip: the Q4_K single-row decode kernel (activation row in LDS)
bool q4k_dec_supported(int k);
void launch_gemv_q4k_dec_f32(const uint8_t* W, int n_out, int k, const float* x, float* y,
                             hipStream_t stream);
void launch_gemv_q4k_dec_ws(const uint8_t* W, int n_out, int k, const uint8_t* ws, float* y,
                            hipStream_t stream);
// The most problems one grouped launch takes.
#define SYN_BATCH 8
void launch_gemv_q4k_batch(int np, const uint8_t* const* W, const int* n_out, const int* k,
                           const uint8_t* const* ws, float* const* y, hipStream_t stream);
void launch_act_quant_batch(int np, const float* const* x, const int* k, uint8_t* const* ws,
                            hipStream_t stream);
// quant.hip
void launch_quantize(int ty, const float* x, uint64_t n, uint8_t* out, hipStream_t stream);
void launch_dequantize(int ty, const uint8_t* src, uint64_t n, float* out, hipStream_t stream);

}  // namespace syn
