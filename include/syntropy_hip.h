/*
 * syntropy_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul and MoE kernels.
 *
 * Plain pointers and sizes only.  Device pointers are HIP device memory; `stream` is a
 * hipStream_t (NULL = the default stream).  Every call only enqueues work on `stream`; it
 * never synchronizes and never allocates device memory.  Each function returns SYN_OK (0)
 * or an error code; the message of the last error on the calling thread is returned by
 * syn_last_error().  A refused call enqueues nothing.
 *
 * Weight types are ggml's type ids: SYN_Q4_0 = 2, SYN_Q8_0 = 8, SYN_Q4_K = 12.  Weights are in
 * GGUF's own block layout, one output row after another (LayoutVersion::SOURCE).
 *
 * Each entry point names the reference interface whose value it computes (paths relative to
 * the reference repository root).  The provider-table boundary the reference's loader binds,
 * `syntropy_provider_entry_v1`, is declared in syntropy_provider.h and is built on these.
 */
#ifndef SYNTROPY_HIP_H
#define SYNTROPY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SYN_OK 0
#define SYN_E_INVALID 1      /* malformed arguments: shape, type, alignment, null pointer */
#define SYN_E_UNSUPPORTED 2  /* a weight type or shape these kernels do not take */
#define SYN_E_WORKSPACE 3    /* the workspace is smaller than the call needs */
#define SYN_E_DEVICE 4       /* the HIP runtime refused the launch */

#define SYN_F16 1
#define SYN_BF16 30
#define SYN_Q4_0 2
#define SYN_Q8_0 8
#define SYN_Q4_K 12

#define SYN_LAYOUT_SOURCE 0 /* the GGUF order */
#define SYN_LAYOUT_X8 1     /* Q4_K runs of eight super-blocks stored chunk-major */
#define SYN_LAYOUT_SPLIT 2  /* Q8_0 / Q4_0: every block's codes, then every block's F16 scale */
#define SYN_LAYOUT_TILE64 3 /* Q4_K rows in runs of 64, each run stored super-block-major */

/* The message of the last failed call on this thread ("" if none). */
const char* syn_last_error(void);
/* Library version: major * 10000 + minor * 100 + patch. */
int syn_version(void);

/* ---- Gemv -------------------------------------------------------------------------------
 * Workspace bytes one syn_gemv call of `rows` activation rows of width `k_in` needs for the
 * quantized activations.  Replaces crates/kernels-cpu/src/gemv/act.rs:108-111
 * (workspace_bytes) as planned by crates/kernels-cpu/src/gemv/entry.rs:68-77. */
int syn_gemv_workspace_bytes(int32_t wtype, uint32_t rows, uint32_t k_in, uint64_t* bytes);

/* Quantizes x F32 [rows, k_in] into the workspace: Q8_0 blocks for Q4_0/Q8_0 weights, Q8_K
 * for Q4_K.  Replaces crates/kernels-cpu/src/gemv/act.rs:122-167 (quantize_into).
 * x: 16-byte aligned; ws: 256-byte aligned. */
int syn_act_quantize(int32_t wtype, const float* x, uint32_t rows, uint32_t k_in, void* ws,
                     uint64_t ws_bytes, void* stream);

/* y F32 [rows, n_out] = W [n_out, k_in] x (activations already quantized into ws by
 * syn_act_quantize for the same wtype, rows and k_in).  Replaces
 * crates/kernels-cpu/src/gemv.rs:435-492 (gemv over every output row). */
int syn_gemv_quantized(int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                       uint32_t k_in, const void* ws, uint64_t ws_bytes, uint32_t rows,
                       float* y, void* stream);

/* The Gemv op: quantize x F32 [rows, k_in], then y F32 [rows, n_out] = W x.  Bit-identical to
 * the reference CPU provider's launch, crates/kernels-cpu/src/gemv/entry.rs:167-247 (run). */
int syn_gemv(int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out, uint32_t k_in,
             const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
             void* stream);

/* ---- Weight layouts ---------------------------------------------------------------------------
 * Layout 1 (X8) of a Q4_K matrix is a permutation of its bytes: each run of eight consecutive
 * 144-byte super-blocks is stored chunk-major (16-byte chunk q of the run's block i at 128 q +
 * 16 i; a final run of m < 8 blocks with stride 16 m).  It needs only the byte count, as the
 * reference's repack does (crates/kernels/src/provider.rs:326-336, repack / repacked_len: the
 * repacked form is the same length).  Decode then reads whole 128-byte lines per load.
 * syn_q4k_repack: on the device (src and dst distinct, 16-byte aligned); inverse = 1 restores
 *   the GGUF order.  syn_q4k_repack_host: the same on host memory.
 * Layout 2 (SPLIT) of a Q8_0 or Q4_0 matrix: the codes of every block in block order (32 bytes
 *   a Q8_0 block, 16 a Q4_0 block), then every block's F16 scale in block order; also the same
 *   length and shape-free.  syn_split_repack(_host) as syn_q4k_repack(_host), for `wtype`.
 * syn_gemv_layout(_workspace_bytes): the Gemv op over a matrix in `layout` (0 is syn_gemv); for
 *   layout 1 one row runs the decode kernel with the row quantized in every workgroup (k_in <=
 *   16384), 2 to 31 rows the decode expert kernel on rows quantized beforehand (int8 matrix
 *   cores, the matrix as one expert) except 2 rows (k_in <= 16384) and 3 or 4 rows (k_in <=
 *   4096), which run the decode kernel over the rows side by side in LDS (with k_in <= 4096 in one
 *   launch that quantizes them in its workgroups); more rows the
 *   matrix-core GEMM (k_in a multiple of 2048).
 *   Layout 2 at one row (k_in up to 39296 for Q4_0, 43680 for Q8_0) is one launch whose
 *   workgroups quantize the row to Q8_0 blocks themselves; otherwise it quantizes the rows to Q8_0 blocks and runs the split decode
 *   kernel eight rows at a time, or the int8 matrix-core GEMM: for k_in a multiple of 128 where
 *   it is the faster (from 2 to 9 rows by shape, always beyond 16), and for Q8_0 of other k_in
 *   from 9 rows.
 * syn_gemv_batch_layout / syn_gemv_batch_quantized_layout: the grouped decode of every problem
 *   in `layout`. */
int syn_q4k_repack(uint32_t layout, const void* src, void* dst, uint64_t bytes, int32_t inverse, void* stream);
int syn_q4k_repack_host(uint32_t layout, const void* src, void* dst, uint64_t bytes, int32_t inverse);
int syn_split_repack(uint32_t layout, int32_t wtype, const void* src, void* dst, uint64_t bytes, int32_t inverse,
                     void* stream);
int syn_split_repack_host(uint32_t layout, int32_t wtype, const void* src, void* dst, uint64_t bytes,
                          int32_t inverse);
int syn_gemv_layout_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t k_in,
                                    uint64_t* bytes);
int syn_gemv_layout(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                    uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                    void* stream);
/* syn_gemv_quantized_layout: the product alone over rows syn_act_quantize quantized for the same
 * wtype (layout 0 is syn_gemv_quantized; layout 2 as syn_gemv_layout without its quantization).
 * Replaces crates/kernels-cpu/src/gemv.rs:435-492 for a repacked matrix. */
int syn_gemv_quantized_layout(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                              uint32_t k_in, const void* ws, uint64_t ws_bytes, uint32_t rows, float* y,
                              void* stream);
/* syn_gemv_layout_noalloc: no counterpart in the reference.  The same Gemv as syn_gemv_layout
 * (same outputs, bit for bit) for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the workspace is a
 * per-device array inside the library, syn_gemv_layout_noalloc_max_workspace() bytes (8 MiB),
 * held until the process ends.  A call whose workspace (syn_gemv_layout_workspace_bytes) is
 * larger is refused with SYN_E_UNSUPPORTED.  It calls no allocator.  Every call on one device
 * shares that device's array: calls that overlap on one device (two streams, two threads) race
 * and must be serialised by the caller. */
uint64_t syn_gemv_layout_noalloc_max_workspace(void);
int syn_gemv_layout_noalloc(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                            uint32_t k_in, const float* x, uint32_t rows, float* y, void* stream);
int syn_gemv_batch_layout(uint32_t layout, uint32_t n, const int32_t* wtypes, const void* const* w,
                          const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                          const float* const* x, float* const* y, void* ws, uint64_t ws_bytes,
                          void* stream);
int syn_gemv_batch_quantized_layout(uint32_t layout, uint32_t n, const int32_t* wtypes, const void* const* w,
                                    const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                                    const void* ws, uint64_t ws_bytes, float* const* y, void* stream);

/* ---- GateUpAct{Silu} -------------------------------------------------------------------------
 * y[r][i] = silu(gate_i . x_r) * (up_i . x_r) for the reference's GateUpAct
 * (crates/kernels/src/reference/linear.rs:75-112), with w one matrix of 2 n_out rows of k_in,
 * gate rows first, then up rows: the ggml provider's binding of the op
 * (crates/kernels-ggml/src/mapping.rs:31).  Each dot is the Gemv value of syn_gemv_layout over
 * the stacked matrix (any row count and layout it serves), silu uses the reference's software
 * exp (crates/kernels/src/reference/math.rs:82-84) and the product is rounded once, as the MoE
 * FFN's gated product (crates/kernels-cpu/src/moe.rs:529-551).  x [rows, k_in] and y
 * [rows, n_out] F32; the workspace holds the Gemv's workspace and the [rows, 2 n_out] product. */
int syn_gate_up_act_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t n_out,
                                    uint32_t k_in, uint64_t* bytes);
int syn_gate_up_act(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                    uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                    void* stream);

/* ---- Measurement (not on the op path) ----------------------------------------------------------
 * syn_hbm_read_probe: reads `bytes` (a multiple of 16, src 16-byte aligned) once with the decode
 * GEMV's load pattern (16-byte non-temporal loads, nine per lane from 256 MiB, one below) and
 * writes one word per workgroup to sink (syn_hbm_read_probe_sink_words(bytes) words): a kernel
 * of known HBM traffic against which the HBM byte counters are calibrated, and a bare read to
 * set a lone op of the same bytes against.  No counterpart in the reference. */
uint64_t syn_hbm_read_probe_sink_words(uint64_t bytes);
int syn_hbm_read_probe(const void* src, uint64_t bytes, uint32_t* sink, void* stream);
/* syn_hbm_read_runs: reads `bytes` once with the X8 decode GEMV's wavefront pattern (a wavefront
 * per 9,216 bytes: nine 16-byte non-temporal loads a lane, instruction i reading line i of eight
 * 1,152-byte runs), `waves` (1 or 8) wavefronts a workgroup; one word per wavefront to sink
 * (syn_hbm_read_runs_sink_words(bytes) words).  The bare read a lone op or the grouped GEMV is
 * set against, beside syn_hbm_read_probe.  No counterpart in the reference. */
uint64_t syn_hbm_read_runs_sink_words(uint64_t bytes);
int syn_hbm_read_runs(uint32_t waves, const void* src, uint64_t bytes, uint32_t* sink, void* stream);
/* syn_div_forms_check: compares, over every F32 bit pattern but the NaNs, the quantizers' short
 * forms of their correctly rounded divisions (amax / 127 for finite amax >= 0, 1 / b, -127 / b),
 * of the F32 -> F16 -> F32 rounding and of ggml's nearest_int (|x| < 2^21) against the
 * compiler's correctly rounded division, the integer F16 conversion and nearest_int's own
 * arithmetic; adds each form's count of differing results to counts[0..4] (device memory, 5
 * words, zero on entry).  A self-check with no counterpart in the reference. */
int syn_div_forms_check(unsigned long long* counts, void* stream);

/* ---- RmsNorm and Logits ----------------------------------------------------------------------
 * syn_rms_norm: y = RmsNorm(x) of each of `rows` rows of n F32 values (n <= 16384), weight g [n]:
 *   ss = sum of x[i] x[i] in the F32Fixed order, mean = ss / n, scale = 1 / sqrt(mean + eps),
 *   y[i] = (x[i] scale) g[i], each one IEEE F32 operation (crates/kernels/src/reference/
 *   norm.rs:39-47; the order crates/kernels/src/reference/reduce.rs:7-20).
 * syn_logits(_workspace_bytes): the reference's Logits (crates/kernels/src/reference/linear.rs:
 *   118-161): each row of x [rows, hidden] normalised as syn_rms_norm (g [hidden], eps), then
 *   the head [vocab, hidden] in `layout` as syn_gemv_layout computes a Gemv, into y [rows, vocab].
 *   The workspace holds the normalised rows and the Gemv's workspace. */
int syn_rms_norm(const float* x, const float* g, uint32_t rows, uint32_t n, float eps, float* y, void* stream);
int syn_logits_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t vocab, uint32_t hidden,
                               uint64_t* bytes);
int syn_logits(uint32_t layout, int32_t wtype, const void* head, uint64_t head_bytes, uint32_t vocab,
               uint32_t hidden, const float* g, float eps, const float* x, uint32_t rows, float* y, void* ws,
               uint64_t ws_bytes, void* stream);

/* ---- Prefill GEMM ---------------------------------------------------------------------------
 * Q4_K weights times many activation rows on the matrix cores, each output bit-identical to
 * syn_gemv (which takes this path itself for Q4_K calls of 32 rows or more).  The reference
 * computes the same value with its Gemv kernel over row groups (crates/kernels-cpu/src/gemv.rs:
 * 435-492; its Gemm kind is Gemv at a larger bucket, crates/kernels/src/reference/linear.rs:
 * 11-13).  k_in must be whole 256-weight super-blocks.
 * syn_gemm_workspace_bytes: the activation workspace for `rows` rows of width k_in.
 * syn_gemm_act_quantize: x F32 [rows, k_in] to Q8_K in the GEMM's layout (x 16-byte, ws
 *   256-byte aligned); the values of crates/kernels-cpu/src/gemv/act.rs:351-373.
 * syn_gemm_q4k_quantized: y F32 [rows, n_out] = W [n_out, k_in] x from that workspace
 *   (w 16-byte aligned). */
int syn_gemm_workspace_bytes(uint32_t rows, uint32_t k_in, uint64_t* bytes);
int syn_gemm_act_quantize(const float* x, uint32_t rows, uint32_t k_in, void* ws, uint64_t ws_bytes,
                          void* stream);
int syn_gemm_q4k_quantized(const void* w, uint64_t w_bytes, uint32_t n_out, uint32_t k_in,
                           const void* ws, uint64_t ws_bytes, uint32_t rows, float* y, void* stream);

/* ---- Grouped decode -----------------------------------------------------------------------
 * Up to 8 independent single-row Q4_K Gemv ops in two launches (one batched Q8_K quantization,
 * one grouped GEMV): y[i] F32 [n_out[i]] = W[i] [n_out[i], k_in[i]] x[i], each bit-identical to
 * syn_gemv on the same operands.  It computes what that many separate calls of the reference's
 * Gemv launch compute (crates/kernels-cpu/src/gemv/entry.rs:167-247); the reference has no
 * grouped form.  Host arrays of n entries; every wtypes[i] must be SYN_Q4_K and every k_in[i]
 * at most 16384.  syn_gemv_batch_workspace_bytes gives the workspace the call needs. */
int syn_gemv_batch_workspace_bytes(uint32_t n, const uint32_t* k_in, uint64_t* bytes);
int syn_gemv_batch(uint32_t n, const int32_t* wtypes, const void* const* w,
                   const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                   const float* const* x, float* const* y, void* ws, uint64_t ws_bytes,
                   void* stream);

/* The two halves of syn_gemv_batch, for callers that quantize once and multiply later (the
 * reference's Gemv launch does the same in two steps: act.rs:122-167, then gemv.rs:435-492):
 * the n rows x[i] (F32 [k_in[i]]) to Q8_K in ws, then the grouped GEMV on ws. */
int syn_act_quantize_batch(uint32_t n, const uint32_t* k_in, const float* const* x, void* ws,
                           uint64_t ws_bytes, void* stream);
int syn_gemv_batch_quantized(uint32_t n, const int32_t* wtypes, const void* const* w,
                             const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                             const void* ws, uint64_t ws_bytes, float* const* y, void* stream);

/* ---- MoE layer ----------------------------------------------------------------------------
 * MoeRoute{Softmax}: ids I32 [rows, top_k] and weights F32 [rows, top_k] from x F32
 * [rows, hidden] and the router F32 [n_experts, hidden].  Logits are F32Fixed dot products
 * (crates/kernels/src/reference/reduce.rs:30-90), softmax subtracts the row maximum and uses the
 * reference's software exp (crates/kernels/src/reference/math.rs:45-75), top-k by probability
 * with the lower expert index on ties, then each selected probability is divided by their
 * in-order sum when `renormalize`.  The reference has no code for this op: it is its
 * specification (plan/rfcs/RFC-0042-quantization-and-numerical-fidelity.md:232,281; the op
 * kind crates/kernels/src/op/kind.rs:35-42, IR signature crates/graph/src/ir/signature.rs:149).
 * probs (F32 [rows, n_experts], required) receives the softmax; the call stages the router
 * logits there first.  Limits: n_experts <= 256, top_k <= min(n_experts, 32), hidden whole
 * 32-value blocks and at most 8192; the router 16-byte aligned. */
int syn_moe_route(const float* router, const float* x, uint32_t rows, uint32_t hidden,
                  uint32_t n_experts, uint32_t top_k, int32_t renormalize, int32_t* ids, float* w,
                  float* probs, void* stream);

/* Packing of the rows*top_k route slots by expert, stable in slot order: offsets u32
 * [n_experts + 1] and slots u32 [rows * top_k], bit-identical to the counting sort of
 * crates/kernels-cpu/src/moe.rs:431-457.  err (device u32[2]): err[0] is 1 when an id is
 * outside [0, n_experts), else 0; err[1] is the largest expert's slot count. */
int syn_moe_pack(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                 uint32_t* offsets, uint32_t* slots, uint32_t* err, void* stream);

/* MoeGrouped: out F32 [rows, top_k, hidden], each slot its expert's SwiGLU FFN of its row
 * alone, bit-identical to crates/kernels-cpu/src/moe.rs:402-551 (moe_grouped) for Q4_K experts.
 * gate, up: [n_experts][inter, hidden] and down: [n_experts][hidden, inter], GGUF Q4_K, stacked
 * by expert (ffn_*_exps); expert_bytes_each is the size of one stacked matrix.  Binding:
 * crates/kernels-cpu/src/moe/entry.rs:6-27.  An id outside [0, n_experts) writes nothing and
 * sets *status (device u32, optional) to 1, as the reference refuses the call
 * (moe.rs:433-441).  site (device I32 [n_experts], optional, MoeGrouped's input 2): a nonzero
 * entry marks an expert this call computes; the slots of the other experts keep their values
 * (entry.rs:13-16, 25, 297-300).  Null: every expert is computed. */
int syn_moe_grouped_workspace_bytes(int32_t wtype, uint32_t n_experts, uint32_t top_k,
                                    uint32_t hidden, uint32_t inter, uint32_t rows,
                                    uint64_t* bytes);
int syn_moe_grouped(int32_t wtype, const void* gate, const void* up, const void* down,
                    uint64_t expert_bytes_each, uint32_t n_experts, uint32_t top_k,
                    uint32_t hidden, uint32_t inter, const float* x, const int32_t* ids,
                    const int32_t* site, uint32_t rows, float* out, void* ws, uint64_t ws_bytes,
                    uint32_t* status, void* stream);

/* Layout 3 (TILE64) of Q4_K rows of k_in values, in whole runs of 64 rows (a matrix, or a stack
 * of matrices such as an MoE layer's experts, of a multiple of 64 rows): within each run, the
 * 144-byte super-block b of the run's row r sits at 144 (64 b + r) from the run's start, so the
 * run's block b is one contiguous 9,216-byte piece.  A permutation of the bytes (the same
 * length, as crates/kernels/src/provider.rs:326-336 asks of a repack), but one that needs k_in:
 * the reference's repack hook receives only the OpKey and the bytes, so the provider keeps MoE
 * experts in GGUF order and this layout is the direct API's.
 * syn_q4k_tile64_repack: on the device (src and dst distinct, 16-byte aligned); inverse = 1
 *   restores the GGUF order.  syn_q4k_tile64_repack_host: the same on host memory.
 * syn_moe_grouped_layout: MoeGrouped over experts in `layout` (0 is syn_moe_grouped; 3 for Q4_K
 *   experts stacked as there, each stack repacked whole), the same bits as over GGUF experts. */
int syn_q4k_tile64_repack(const void* src, void* dst, uint64_t bytes, uint32_t k_in, int32_t inverse, void* stream);
int syn_q4k_tile64_repack_host(const void* src, void* dst, uint64_t bytes, uint32_t k_in, int32_t inverse);
int syn_moe_grouped_layout(uint32_t layout, int32_t wtype, const void* gate, const void* up, const void* down,
                           uint64_t expert_bytes_each, uint32_t n_experts, uint32_t top_k, uint32_t hidden,
                           uint32_t inter, const float* x, const int32_t* ids, const int32_t* site, uint32_t rows,
                           float* out, void* ws, uint64_t ws_bytes, uint32_t* status, void* stream);

/* MoeCombine: y F32 [rows, hidden] = per row, the slots of out F32 [rows, top_k, hidden] in
 * ascending expert id, y += w * v from +0.0 without fused multiply-add
 * (crates/kernels-cpu/src/moe/tests.rs:541-556; IR signature
 * crates/graph/src/ir/signature.rs:153). */
int syn_moe_combine(const float* out, const int32_t* ids, const float* w, uint32_t rows,
                    uint32_t top_k, uint32_t hidden, float* y, void* stream);

/* MoeCombine as the graph binds it: inputs [per_expert, weights, shared...], dims [top_k,
 * n_shared, hidden] (crates/kernels/src/op/kind.rs:244; crates/graph/src/ir/signature.rs:153;
 * crates/graph/src/blocks/ffn.rs:189-200).  The binding carries no expert ids, so the slots of
 * out F32 [rows, top_k, hidden] are added in rank order (slot j = rank j, the order MoeRoute
 * writes; plan/rfcs/RFC-0042-quantization-and-numerical-fidelity.md:233), then each of the
 * n_shared <= 8 shared outputs F32 [rows, hidden] (shared: a host array of device pointers):
 * y = 0.0, y += w_j * v_j, y += shared_s, in F32 without fused multiply-add. */
int syn_moe_combine_ranked(const float* out, const float* w, uint32_t n_shared,
                           const float* const* shared, uint32_t rows, uint32_t top_k, uint32_t hidden,
                           float* y, void* stream);

/* ---- MoE residency split --------------------------------------------------------------------
 * The doorbell layer a router op writes and the split rule every site evaluates from it
 * (plan/rfcs/RFC-0040-kernel-providers-and-backends.md:380-403; RFC-0023 sections 2 and 6).
 * Layouts and codes are those of crates/kernels/include/syntropy/moe_doorbell.h (ABI version 1):
 * a layer is the 8-byte header { u32 seq; u16 n_route; u16 n_pred }, then route[max_union] of
 * 8-byte { u16 expert; u16 tokens; u32 cache_slot } entries, then the predictions, all
 * little-endian. */
#define SYN_MOE_MISS 4294967295u /* cache_slot of an expert not in the device's cache */
#define SYN_MOE_HIT 4294967295u  /* code: computed from its cache slot */
#define SYN_MOE_CPU 4294967294u  /* code: computed in place by the CPU pools; below it: copy slot */

/* The doorbell layer of one pass (RFC-0040 ...md:390): seq, then one route entry per distinct
 * expert of ids I32 [rows, top_k], in ascending expert index, tokens = the rows that selected it,
 * cache_slot = slot_of[expert] (device u32 [n_experts], the slot_of table of RFC-0040 ...md:384;
 * null: every expert misses); n_pred = 0 and the prediction part is not written.  step_desc
 * (device syn_step_desc, optional): seq is the low 32 bits of its step and its rows_active
 * bounds the rows, both read on the device; without it, seq is the argument.  status (device
 * u32, optional): 0; 1 for an id outside [0, n_experts); 2 when the distinct experts exceed
 * max_union (DoorbellError::TooManyRoutes, crates/kernels/src/moe/doorbell.rs:17); the layer
 * is written only with status 0.  Limits: n_experts <= 8192, top_k <= 32, rows <= 65535; the
 * layer 8-byte aligned. */
int syn_moe_doorbell(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                     const uint32_t* slot_of, const void* step_desc, uint32_t seq, void* layer,
                     uint32_t max_union, uint32_t* status, void* stream);

/* The split rule, bit-identical to syn_moe_assign of crates/kernels/include/syntropy/
 * moe_assign.h:29-61 (crates/kernels/src/moe.rs:110-160 assign_into): out[i] (device u32) is
 * SYN_MOE_HIT for a hit; for a miss marked in eligible (bit e % 32 of word e / 32, for e below
 * n_experts), copy slot c, its rank among such misses ordered by tokens descending, expert
 * ascending, then entry, while c < copy_slots and (c + 1) * expert_bytes <= b_copy; SYN_MOE_CPU
 * otherwise.  route: device entries as above, 8-byte aligned; n_route <= 65535. */
int syn_moe_assign(const void* route, uint32_t n_route, const uint32_t* eligible, uint32_t n_experts,
                   uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots, uint32_t* out,
                   void* stream);

/* The same over a doorbell layer, every input read on the device (so that a captured graph
 * follows the step): n_route from its header (a header above max_union writes no code, as
 * DoorbellLayer::read refuses it, doorbell.rs:326-340), b_copy from the device word b_copy (the
 * step descriptor's moe_balance entry of the layer, step_desc.h:85-87).  Codes past n_route are
 * not written. */
int syn_moe_assign_layer(const void* layer, uint32_t max_union, const uint32_t* eligible,
                         uint32_t n_experts, const uint32_t* b_copy, uint64_t expert_bytes,
                         uint32_t copy_slots, uint32_t* out, void* stream);

/* site I32 [n_experts] = 1 for the experts of the layer's route whose code is of class `which`
 * (0 HIT, 1 COPY, 2 CPU), 0 for all others: MoeGrouped's site input for that class's launch
 * (crates/kernels-cpu/src/moe/entry.rs:13-16).  No reference counterpart: the glue between the
 * codes and the site mask. */
int syn_moe_site_mask(const void* layer, uint32_t max_union, const uint32_t* codes, uint32_t n_experts,
                      int32_t which, int32_t* site, void* stream);

/* ---- Weight packing ---------------------------------------------------------------------
 * x F32 [n] -> GGUF blocks of wtype, byte-identical to ggml's reference quantizers
 * (third_party/ggml/src/ggml-quants.c:113-140, 276-297, 1458-1528, wrapped by
 * crates/kernels-ggml/src/lib.rs:268 quantize).  n must be whole blocks; the caller checks
 * that every value is finite and at most 65504 in magnitude, as that wrapper does. */
int syn_quantize(int32_t wtype, const float* x, uint64_t n, void* out, uint64_t out_bytes,
                 void* stream);

/* GGUF blocks -> F32, exact (crates/kernels/src/reference/dequant.rs:195-229). */
int syn_dequantize(int32_t wtype, const void* src, uint64_t src_bytes, float* out,
                   void* stream);

#ifdef __cplusplus
}
#endif
#endif
