/*
 * oracle.h -- CPU restatement of the reference's quantized-matmul and MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is what the HIP path is compared against
 * (and the "port" CPU baseline that bench.py times).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function restates, operation for operation, the reference function named in its
 * comment (paths are relative to the reference repository root).  Where the reference has no
 * code (MoeRoute, MoeCombine) the comment names the specification followed instead.
 */
#ifndef SYNTROPY_ORACLE_H
#define SYNTROPY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (ggml's enum ggml_type values). */
enum {
    OR_F32 = 0,
    OR_F16 = 1,
    OR_Q4_0 = 2,
    OR_Q8_0 = 8,
    OR_Q4_K = 12,
    OR_BF16 = 30,
};

/* Activation block kinds (crates/kernels-cpu/src/gemv/act.rs:31-39). */
enum { OR_ACT_F32 = 0, OR_ACT_Q8_0 = 1, OR_ACT_Q8K = 2 };

/* ---- scalar conversions (crates/kernels/src/reference/act_quant.rs:398-485) ---- */
uint16_t or_f16_bits(float x);
float or_f16_to_f32(uint16_t h);
uint16_t or_round_bf16(float x);
float or_bf16_to_f32(uint16_t h);

/* ---- software exp / silu (crates/kernels/src/reference/math.rs:45-84) ---- */
float or_exp(float x);
float or_silu(float x);
double or_exp_worst_ulp(uint32_t step);

/* ---- F32Fixed reductions (crates/kernels/src/reference/reduce.rs:30-90) ---- */
float or_sum(const float* xs, size_t n);
float or_dot(const float* a, const float* b, size_t n);

/* ---- block geometry (crates/kernels/src/reference/dequant.rs:46-84) ---- */
int or_block_elems(int ty);
int or_block_bytes(int ty);
int or_act_kind(int ty); /* crates/kernels-cpu/src/gemv.rs:145-151 */

/* ---- exact dequant (crates/kernels/src/reference/dequant.rs:133-173, 195-229) ---- */
int or_dequantize(int ty, const uint8_t* src, size_t nbytes, float* out);

/* ---- weight quantizers, ggml's quantize_row_*_ref
 *      (third_party/ggml/src/ggml-quants.c:113-140, 276-297, 621-626, 799-878, 1458-1528);
 *      F16/BF16 rows are ggml's row conversions.  Returns bytes written or -1. ---- */
long or_quantize(int ty, const float* x, size_t n, uint8_t* out);

/* ---- reference activation quantizers in ggml's byte layouts
 *      (crates/kernels/src/reference/act_quant.rs:241-393).
 *      path: 0 = Reference (roundf), 1 = Arm64Neon (ties even), 2 = X86Avx.  ---- */
int or_quantize_q8_0_blocks(const float* x, size_t n, int path, uint8_t* out);
int or_quantize_q8_1_blocks(const float* x, size_t n, int path, uint8_t* out);
int or_quantize_q8_k_blocks(const float* x, size_t n, uint8_t* out);

/* ---- GEMV activation workspace (crates/kernels-cpu/src/gemv/act.rs:98-167):
 *      [scales f32 | sums i32 | codes i8].  ---- */
size_t or_act_workspace_bytes(int kind, size_t rows, size_t k);
int or_act_quantize(int kind, const float* x, size_t rows, size_t k, uint8_t* ws);

/* ---- GEMV (crates/kernels-cpu/src/gemv.rs:435-492, gemv/portable.rs:15-190):
 *      y[r][o] for o in [o_begin, o_end) from quantized activations in ws. ---- */
int or_gemv_ws(int ty, const uint8_t* w, size_t n_out, size_t k, const uint8_t* ws,
               const float* xf, size_t rows, size_t o_begin, size_t o_end, float* y);
/* quantize + gemv over all outputs; ws may be NULL (allocated internally) */
int or_gemv(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows,
            float* y);
/* the same, split over `threads` pthreads by the reference's partition (gemv.rs:402-421) */
int or_gemv_threads(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x,
                    size_t rows, float* y, int threads);
int or_gate_up_act(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows,
                   float* y, int threads);
void or_partition(int ty, size_t n_out, size_t k, size_t parts, size_t* starts, size_t* ends);

/* ---- RmsNorm (crates/kernels/src/reference/norm.rs:39-47) and Logits
 *      (crates/kernels/src/reference/linear.rs:118-161): rows normalised, then the head as Gemv ---- */
void or_rms_norm_row(const float* x, const float* g, size_t n, float eps, float* y);
int or_rms_norm(const float* x, const float* g, size_t rows, size_t n, float eps, float* y);
int or_logits(int ty, const uint8_t* head, size_t vocab, size_t hidden, const float* g, float eps,
              const float* x, size_t rows, float* y, int threads);

/* ---- MoE (crates/kernels-cpu/src/moe.rs:402-551) ---- */
size_t or_moe_workspace_bytes(size_t n_experts, size_t top_k, size_t hidden, size_t inter,
                              size_t rows);
/* Counting-sort packing: offsets[n_experts+1], slots[rows*top_k].  -1 on a bad id. */
/* The reference's x86 level (crates/kernels-cpu/src/gemv/x86.rs; ROW_GROUP = 8 rows a weight
 * pass): the same outputs as or_gemv_threads / or_moe_grouped, timed as the CPU baseline. */
int or_gemv_x86(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows, float* y,
                int threads);
int or_moe_grouped_x86(int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                       size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                       float* out, int threads);
int or_moe_pack(const int32_t* ids, size_t rows, size_t top_k, size_t n_experts,
                uint32_t* offsets, uint32_t* slots);
/* site: NULL (every expert) or n_experts ints, nonzero = computed here. */
int or_moe_grouped(int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                   size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                   const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                   float* out, int threads);

/* ---- MoeRoute{Softmax} (spec: plan/rfcs/RFC-0042-...md:232,281; RFC-0040 ...md:294,848) ---- */
int or_moe_route(const float* router, const float* x, size_t rows, size_t hidden,
                 size_t n_experts, size_t top_k, int renormalize, int32_t* ids, float* weights,
                 float* probs /* optional [rows, n_experts] */);

/* ---- MoeCombine (crates/kernels-cpu/src/moe/tests.rs:541-556) ---- */
int or_moe_combine(const float* out, const int32_t* ids, const float* w, size_t rows,
                   size_t top_k, size_t hidden, float* y);
/* ---- MoeCombine as the IR binds it (crates/kernels/src/op/kind.rs:244;
 * crates/graph/src/ir/signature.rs:153): slots in rank order, then the shared experts'
 * outputs ([n_shared][rows][hidden]); RFC-0042 ...md:233 ---- */
int or_moe_combine_ranked(const float* out, const float* w, const float* shared, size_t n_shared,
                          size_t rows, size_t top_k, size_t hidden, float* y);

/* ---- The residency split: doorbell layer and split rule
 * (crates/kernels/include/syntropy/moe_doorbell.h, moe_assign.h; RFC-0040 ...md:380-403) ---- */
#define OR_MOE_MISS 0xFFFFFFFFu
#define OR_MOE_HIT 0xFFFFFFFFu
#define OR_MOE_CPU 0xFFFFFFFEu
struct or_route_slot {
    uint16_t expert;
    uint16_t tokens;
    uint32_t cache_slot;
};
void or_moe_assign(const struct or_route_slot* route, uint32_t n_route, const uint32_t* eligible,
                   uint32_t n_experts, uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots,
                   uint32_t* out);
/* The doorbell layer (header, then route[max_union]) of one pass: -1 for an id outside
 * [0, n_experts), -2 when the distinct experts exceed max_union; the layer is untouched then. */
int or_moe_doorbell(const int32_t* ids, size_t rows, size_t top_k, uint32_t n_experts,
                    const uint32_t* slot_of /* optional */, uint32_t seq, uint32_t max_union,
                    uint8_t* layer);

/* ---- seeded generators (SplitMix64 + Box-Muller, for the synthetic workloads) ---- */
void or_normal_f32(uint64_t seed, float sigma, float* out, size_t n);

/* ---- helpers ---- */
uint64_t or_fnv1a(const uint8_t* bytes, size_t n);
int or_num_threads_default(void);

#ifdef __cplusplus
}
#endif
#endif
