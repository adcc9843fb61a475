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
                   float* y, hipStream_t stream, const uint32_t* active = nullptr);
// gemv_q4k.hip: the Q4_K single-row decode kernel (activation row in LDS)
bool q4k_dec_supported(int k);
// Q4_K at 2 to 4 rows over X8 weights, where gemv_q4k_x8_rows_pick finds it the faster form, on
// Q8_K rows quantized by launch_act_quant
bool gemv_q4k_x8_rows_pick(int n_out, int k, int rows);
// with x (F32 rows, not ws) where gemv_q4k_x8_rows_fused(k, rows): the rows quantized in the
// workgroups
bool gemv_q4k_x8_rows_fused(int k, int rows);
void launch_gemv_q4k_x8_rows(const uint8_t* W, int n_out, int k, const uint8_t* ws, const float* x, int rows,
                             float* y, hipStream_t stream, const uint32_t* active);
void launch_gemv_q4k_dec_f32(const uint8_t* W, int n_out, int k, const float* x, float* y,
                             hipStream_t stream, const uint32_t* active = nullptr);
void launch_gemv_q4k_dec_ws(const uint8_t* W, int n_out, int k, const uint8_t* ws, float* y,
                            hipStream_t stream);
// The most problems one grouped launch takes.
#define SYN_BATCH 8
void launch_gemv_q4k_batch(int layout, int np, const uint8_t* const* W, const int* n_out, const int* k,
                           const uint8_t* const* ws, float* const* y, hipStream_t stream);
// Gemv over F16 / BF16 weights (F32 activations, 32 FMA accumulators and the halving fold).
void launch_gemv_float(int ty, const uint8_t* W, int n_out, int k, const float* x, int rows, float* y,
                       hipStream_t stream, const uint32_t* active = nullptr);
// GateUpAct{Silu}'s gated product over the Gemv of the stacked [gate; up] weight.
void launch_silu_mul(const float* y2, int rows, int n, float* y, hipStream_t stream, const uint32_t* active = nullptr);
// The same over X8 weights with the F32 rows quantized inside the grouped launch (k <= 16384).
bool gemv_q4k_batch_fusable(int k);
// 2..8 rows over X8 weights, the rows quantized beforehand (act_layout(ACT_Q8K, rows, k) at ws)
// GateUpAct{Silu} at one row over a stacked [gate; up] X8 matrix of 2 n rows: y[i] = silu(g_i) * u_i
void launch_gate_up_q4k_f32(const uint8_t* W, int n, int k, const float* x, float* y, hipStream_t stream,
                            const uint32_t* active = nullptr);
void launch_gemv_q4k_batch_f32(const uint8_t* const* W, int np, const int* n_out, const int* k,
                               const float* const* x, float* const* y, hipStream_t stream,
                               const uint32_t* active = nullptr);
// The X8 repack of a Q4_K matrix of nblocks super-blocks (inverse = 1: back to the GGUF order).
void launch_q4k_x8(const uint8_t* src, uint8_t* dst, uint64_t nblocks, int inverse, hipStream_t stream);
void launch_act_quant_batch(int np, const float* const* x, const int* k, uint8_t* const* ws,
                            hipStream_t stream);
// moe_q8.hip: MoeGrouped over Q8_0 experts (Q8_0 entries' rows, gate/up + silu, down)
void launch_moe_gather_q8_0(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                            const uint32_t* err, int8_t* codes, float* d, int gather, const uint32_t* total,
                            hipStream_t stream);
void launch_moe_q8(int mode, const uint8_t* w0, const uint8_t* w1, uint64_t mat_bytes, int n_experts, int n_out,
                   int k, const uint32_t* offsets, const uint32_t* slots, const uint32_t* err, const int8_t* aq,
                   const float* ad, float* y, hipStream_t stream);
// gemv_split.hip: Q8_0 / Q4_0 in the SPLIT layout (codes, then scales); activations Q8_0 rows
void launch_split_repack(int ty, const uint8_t* src, uint8_t* dst, uint64_t bytes, int inverse, hipStream_t stream);
void launch_gemv_split(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int rows, float* y,
                       hipStream_t stream, const uint32_t* active = nullptr);
void launch_gemm_q8_split(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int T, float* y,
                          hipStream_t stream, const uint32_t* active = nullptr);
bool gemm_q8_staged_fits(int ty, int n_out, int k, int T);
bool gemm_q8_splitk_fits(int ty, int n_out, int k, int T);
// estimated microseconds of the int8 GEMM launch_gemm_q8_split picks (gemv_split.hip)
double gemm_q8_cost_us(int ty, int n_out, int k, int T);
bool gemv_split_staged(int ty, int rows, int k);
bool gemv_split_fused_fits(int ty, int k);
void launch_gemv_split_fused(int ty, const uint8_t* W, int n_out, int k, const float* x, float* y, hipStream_t stream,
                             const uint32_t* active);
// probe.hip: a read-only HBM stream with the decode GEMV's load pattern (counter calibration)
void launch_hbm_read_probe(const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream);
uint64_t hbm_read_probe_workgroups(uint64_t bytes);
uint64_t hbm_read_runs_units(uint64_t bytes);
void launch_hbm_read_runs(int waves, const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream);
void launch_div_forms_check(unsigned long long* counts, hipStream_t stream);
// norm.hip: RmsNorm rows of at most NORM_MAX_COLS values
constexpr int NORM_MAX_COLS = 16384;
void launch_rms_norm(const float* x, const float* g, int rows, int n, float eps, float* y, hipStream_t stream,
                     const uint32_t* active = nullptr);
// moe.hip
bool moe_route_supported(int hidden);
void launch_moe_route(const float* router, const float* x, int rows, int hidden, int n_experts,
                      int top_k, int renorm, int32_t* ids, float* w, float* probs, float* logits,
                      hipStream_t stream, const uint32_t* active = nullptr);
void launch_moe_pack(const int32_t* ids, int nslots, int n_experts, uint32_t* offsets,
                     uint32_t* slots, uint32_t* err, hipStream_t stream, const uint32_t* active = nullptr, int top_k = 1,
                     const int32_t* site = nullptr, uint32_t* report = nullptr);
// Q8_K activations of the packed entries as the expert kernels read them, entry-major.  Each
// 256-value block b of an entry is stored in the matrix-core operand order: byte
// 256b + 64p + 16(j%4) + 8(j/4) + i holds code 32j + 8p + i (sub-block j, k part p), so that
// one lane reads its A operand of all eight sub-blocks as 64 contiguous bytes, the two
// sub-blocks j and j + 4 it multiplies together side by side.  lh holds, per block, the
// sub-block code sums s_j = 128 h_j + l_j as bytes l_0..l_7 (0..127), h_0..h_7 (-32..31).
struct MoeAct {
    int8_t* codes;  // [entry][k]
    float* d;       // [k / 256][dstride] (block-major, rows padded to 4 entries)
    uint8_t* lh;    // [entry][k / 256][16]
    int nentries;
    int dstride;
};
size_t moe_act_bytes(int64_t nentries, int k);
MoeAct moe_act_at(uint8_t* base, int64_t nentries, int k);
void launch_moe_gather_q8k(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                           const uint32_t* err, MoeAct a, int gather, hipStream_t stream, const uint32_t* total = nullptr);
void launch_moe_gateup(const uint8_t* gate, const uint8_t* up, int n_experts, int hidden,
                       int inter, const uint32_t* offsets, int nentries, MoeAct a,
                       const uint32_t* err, float* h, hipStream_t stream, int layout);
void launch_q4k_dense_rows(const uint8_t* W, int x8, int n_out, int k, MoeAct a, int rows, float* y,
                           hipStream_t stream, const uint32_t* active = nullptr);
void launch_moe_down(const uint8_t* down, int n_experts, int hidden, int inter,
                     const uint32_t* offsets, int nentries, MoeAct a, const uint32_t* slots,
                     const uint32_t* err, float* out, hipStream_t stream, int layout);
void launch_moe_combine(const float* out, const int32_t* ids, const float* w, int rows, int top_k,
                        int hidden, float* y, hipStream_t stream, const uint32_t* active = nullptr);
// The shared experts' outputs MoeCombine adds after the routed slots, [rows, hidden] each.
constexpr int MAX_SHARED = 8;
struct SharedOuts {
    const float* p[MAX_SHARED];
    int n;
};
void launch_moe_combine_ranked(const float* out, const float* w, const SharedOuts& sh, int rows, int top_k,
                               int hidden, float* y, hipStream_t stream, const uint32_t* active = nullptr);
// moe_split.hip: the residency split (doorbell layer, split rule, site masks)
void launch_moe_assign(const uint8_t* route, uint32_t n_route, const uint32_t* eligible, uint32_t n_experts,
                       uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots, uint32_t* out,
                       hipStream_t stream);
void launch_moe_assign_layer(const uint8_t* layer, uint32_t max_union, const uint32_t* eligible,
                             uint32_t n_experts, const uint32_t* b_copy, uint64_t expert_bytes,
                             uint32_t copy_slots, uint32_t* out, hipStream_t stream);
void launch_moe_doorbell(const int32_t* ids, int rows, int top_k, int n_experts, const uint32_t* slot_of,
                         const void* desc, uint32_t seq, uint8_t* layer, uint32_t max_union, uint32_t* status,
                         hipStream_t stream);
void launch_moe_site_mask(const uint8_t* layer, uint32_t max_union, const uint32_t* codes, int n_experts,
                          int which, int32_t* site, hipStream_t stream);
// doorbell.hip: the device halves of the host <-> device flags (a bounded wait)
void launch_bell_signal(uint32_t* flag, uint32_t value, hipStream_t stream);
void launch_bell_wait(uint32_t* flag, uint32_t value, int geq, int has_reset, uint32_t reset, uint64_t max_ticks,
                      uint32_t* status, uint32_t tag, hipStream_t stream);
// gemm_q4k.hip: the prefill Q4_K GEMM on the F16 matrix cores.  Activations are quantized to
// Q8_K into the GEMM's own layout (codes as F16 in the matrix-core operand order, then per
// super-block the sub-block sums, scales and block sums); tpad = rows rounded up to 64.
struct GemmAct {
    uint8_t* codes;
    uint8_t* tail;
    int tpad;
};
size_t gemm_act_bytes(int64_t tpad, int k);
GemmAct gemm_act_at(uint8_t* base, int64_t tpad, int k);
void launch_gemm_act(const float* x, int T, int k, GemmAct a, hipStream_t stream, const uint32_t* active = nullptr);
bool gemm_q4k_supported(int n_out, int k);
void launch_gemm_q4k(int layout, const uint8_t* W, int n_out, int k, GemmAct a, int T, float* y, hipStream_t stream,
                     const uint32_t* active = nullptr);
// The MoE expert FFN at many tokens on the same kernels: entries padded to 64-entry tiles per
// expert (pad_off [E+1], tile_e [max_tiles], n_tiles [1], built on the device from the packed
// offsets); gate/up -> h on the tokens' rows quantized once (launch_gemm_act) and gathered per
// position, then down -> the slots on h quantized at the padded positions.
struct MoeTiles {
    uint32_t* pad_off;
    uint32_t* tile_e;
    uint32_t* n_tiles;
};
bool moe_gemm_supported(int hidden, int inter);
void launch_moe_tiles(const uint32_t* offsets, int n_experts, const uint32_t* err, MoeTiles mt, hipStream_t stream);
void launch_moe_gemm_act(const float* h, int k, const uint32_t* offsets, MoeTiles mt, const uint32_t* err,
                         GemmAct a, hipStream_t stream);
// mode 0 (gate/up): act holds the tokens' rows (launch_gemm_act of x), gathered per position;
// mode 1 (down): act holds the entries' h rows at their padded positions.  The experts in GGUF
// order or TILE64 (`layout`).
void launch_moe_gemm(int mode, const uint8_t* w0, const uint8_t* w1, int n_experts, int rows, int k,
                     GemmAct act, int max_tiles, const uint32_t* offsets, MoeTiles mt, const uint32_t* err,
                     const uint32_t* slots, float* out, hipStream_t stream, int top_k, int layout);
// TILE64 <-> GGUF order of `bytes` of Q4_K rows of k values (whole 64-row runs).
void launch_tile64_repack(const uint8_t* src, uint8_t* dst, uint64_t bytes, int k, int inverse, hipStream_t stream);
// quant.hip
void launch_quantize(int ty, const float* x, uint64_t n, uint8_t* out, hipStream_t stream);
void launch_dequantize(int ty, const uint8_t* src, uint64_t n, float* out, hipStream_t stream);

}  // namespace syn
