/*
 * ref_driver.c -- TEST INFRASTRUCTURE.  Thin C-ABI over the reference's vendored ggml
 * quantizers, so tests can compare the oracle's restatement with ggml's own code.
 *
 * Compiled together with third_party/ggml/src/ggml-quants.c where the reference tree is
 * present (oracle/Makefile, target `ref`); the output goes to oracle/_ref/ only.  No ggml
 * source is copied into this repository.
 */
#include <stddef.h>
#include <stdint.h>

#include "ggml-common.h"
#include "ggml-quants.h"

#define REF_API __attribute__((visibility("default")))

/* ggml type ids: Q4_0 = 2, Q8_0 = 8, Q4_K = 12 */
REF_API int ref_quantize(int ty, const float* x, int64_t n, void* out) {
    switch (ty) {
    case 2: quantize_row_q4_0_ref(x, (block_q4_0*)out, n); return 0;
    case 8: quantize_row_q8_0_ref(x, (block_q8_0*)out, n); return 0;
    case 12: quantize_row_q4_K_ref(x, (block_q4_K*)out, n); return 0;
    default: return -1;
    }
}

REF_API int ref_dequantize(int ty, const void* src, int64_t n, float* out) {
    switch (ty) {
    case 2: dequantize_row_q4_0((const block_q4_0*)src, out, n); return 0;
    case 8: dequantize_row_q8_0((const block_q8_0*)src, out, n); return 0;
    case 12: dequantize_row_q4_K((const block_q4_K*)src, out, n); return 0;
    default: return -1;
    }
}

/* ggml's activation quantizers: 0 = quantize_row_q8_0_ref, 1 = quantize_row_q8_1_ref,
 * 2 = quantize_row_q8_K_ref */
REF_API int ref_quantize_act(int which, const float* x, int64_t n, void* out) {
    switch (which) {
    case 0: quantize_row_q8_0_ref(x, (block_q8_0*)out, n); return 0;
    case 1: quantize_row_q8_1_ref(x, (block_q8_1*)out, n); return 0;
    case 2: quantize_row_q8_K_ref(x, (block_q8_K*)out, n); return 0;
    default: return -1;
    }
}
