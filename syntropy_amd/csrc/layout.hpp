// Host-side geometry of the path: GGUF block sizes and the layout of the quantized
// activations the GEMV kernels read.
#pragma once

#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define SYN_HD __host__ __device__
#else
#define SYN_HD
#endif

namespace syn {

// GGUF type ids (ggml's enum ggml_type values).
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_BF16 = 30 };
// Activation block kinds (crates/kernels-cpu/src/gemv/act.rs:31-39).
enum : int { ACT_F32 = 0, ACT_Q8_0 = 1, ACT_Q8K = 2 };

inline int block_elems(int ty) {
    switch (ty) {
    case 1: case 30: return 1;     // F16, BF16
    case 2: case 8: return 32;     // Q4_0, Q8_0
    case 12: return 256;           // Q4_K
    default: return 0;
    }
}
inline int block_bytes(int ty) {
    switch (ty) {
    case 1: case 30: return 2;
    case 2: return 18;
    case 8: return 34;
    case 12: return 144;
    default: return 0;
    }
}
// The activation block a product over weight type `ty` quantizes to
// (crates/kernels-cpu/src/gemv.rs:145-151): Q8_0 for Q8_0/Q4_0, Q8_K for Q4_K.
inline int act_kind(int ty) {
    switch (ty) {
    case 2: case 8: return 1;
    case 12: return 2;
    default: return 0;
    }
}
SYN_HD inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Quantized activations of `rows` rows of `k` values in device memory.  The provider owns
// this layout (the workspace is provider-declared scratch): codes first, then one F32 scale
// per block, then one I32 code sum per 32 values; each section starts on 256 bytes.
//   kind 1 (Q8_0): scale per 32 values; sums feed Q4_0's offset-8 term.
//   kind 2 (Q8_K): scale per 256 values; sums feed Q4_K's minimum term.
struct ActLayout {
    uint64_t codes, d, sums, bytes;
};
SYN_HD inline ActLayout act_layout(int kind, uint64_t rows, uint64_t k) {
    ActLayout l{0, 0, 0, 0};
    if (kind == 0) return l;
    uint64_t n = rows * k;
    uint64_t nd = kind == 1 ? n / 32 : n / 256;
    l.codes = 0;
    l.d = align_up(n, 256);
    l.sums = align_up(l.d + 4 * nd, 256);
    l.bytes = align_up(l.sums + 4 * (n / 32), 256);
    return l;
}

// Weight layouts of Q4_K matrices (the OpKey's LayoutVersion).
//  0 SOURCE: the GGUF order, 144-byte super-blocks one after the other.
//  1 X8: the same bytes with each run of eight consecutive super-blocks (1152 bytes) stored
//    chunk-major: 16-byte chunk q of the run's block i at 128 q + 16 i.  A final run of m < 8
//    blocks is stored the same way with stride 16 m.  Shape-free (a permutation of the matrix
//    bytes), so a repack needs only the byte count.
//  2 SPLIT (Q8_0 and Q4_0 matrices): the codes of every block in block order (32 bytes a block
//    for Q8_0, 16 for Q4_0), then every block's F16 scale in block order.  Also shape-free: block
//    g's codes sit at cb g and its scale at cb nblocks + 2 g (cb = 32 or 16).
//  3 TILE64 (Q4_K matrices of whole 64-row runs, and stacks of them such as an MoE layer's
//    experts): within each run of 64 consecutive rows, super-block b of the run's row r sits at
//    144 (64 b + r) from the run's start, so the 64 rows' block b is one contiguous 9,216-byte
//    piece.  A permutation of the matrix bytes that needs the row length besides the byte count.
enum : int { LAYOUT_SOURCE = 0, LAYOUT_X8 = 1, LAYOUT_SPLIT = 2, LAYOUT_TILE64 = 3 };
constexpr int TILE64_ROWS = 64;
// Byte offset of row r's super-block 0 in a TILE64 matrix of rb-byte rows (block b adds 9216 b).
SYN_HD inline uint64_t tile64_row_offset(uint64_t r, uint64_t rb) {
    return (r / TILE64_ROWS) * TILE64_ROWS * rb + (r % TILE64_ROWS) * 144;
}
SYN_HD inline int split_code_bytes(int ty) { return ty == T_Q8_0 ? 32 : 16; }
SYN_HD inline uint32_t x8_group_blocks(uint64_t g, uint64_t nblocks) {
    const uint64_t first = g & ~(uint64_t)7;
    return nblocks - first < 8 ? (uint32_t)(nblocks - first) : 8u;
}
// Byte offset of chunk q (0..8) of super-block g in an X8 matrix of nblocks blocks.
SYN_HD inline uint64_t x8_chunk_offset(uint64_t g, int q, uint64_t nblocks) {
    const uint64_t first = g & ~(uint64_t)7;
    return first * 144 + 16 * ((uint64_t)q * x8_group_blocks(g, nblocks) + (g - first));
}

}  // namespace syn
