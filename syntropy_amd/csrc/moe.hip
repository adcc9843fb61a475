// The MoE layer on gfx950: MoeRoute{Softmax}, token-to-expert packing, the grouped expert
// SwiGLU FFN (MoeGrouped) and MoeCombine.
//
// Values:
//  * route: logits as F32Fixed dot products (crates/kernels/src/reference/reduce.rs:30-90: 32-term
//    blocks summed in order, then the level-by-level pairwise tree), softmax with the row maximum
//    subtracted, the reference's software exp and an F32Fixed sum; top-k by probability, lower
//    expert index on ties; renormalized by the in-order sum of the k selected probabilities.
//    The reference has no code for this op; this is its specification
//    (plan/rfcs/RFC-0042-quantization-and-numerical-fidelity.md:232,281).
//  * pack: crates/kernels-cpu/src/moe.rs:431-457, a counting sort of the slots r*k+j by expert,
//    stable in slot order.  Bit-exact.
//  * grouped FFN: crates/kernels-cpu/src/moe.rs:470-551 for Q4_K experts: every slot's output is
//    its expert's FFN of its row alone, h = silu(gate x) * (up x), h requantized to Q8_K, then
//    down h; each product is the Gemv value of crates/kernels-cpu/src/gemv.rs (exact per
//    sub-block I32 sums, one F32 term per super-block, terms folded in super-block order).
//  * combine: crates/kernels-cpu/src/moe/tests.rs:541-556: per row, the slots in ascending
//    expert id, y += w * v in F32 from +0.0, no fused multiply-add.
//
// The expert products run on the int8 matrix cores: v_mfma_i32_16x16x32_i8 computes, for one
// 32-value sub-block, the exact I32 sums of 16 tokens (A) against 16 weight rows (B).  The k
// order inside a sub-block is free (the sums are exact), so each lane feeds the 8 codes of its
// own 8 packed bytes.  The F32 epilogue per (row, token, super-block) applies the 6-bit scales
// and minimums and folds in super-block order, in the lane that owns the output.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ============================================================================================
// MoeRoute{Softmax}
// ============================================================================================

// Logits: one workgroup per (RT_T tokens, RT_E experts), walking the hidden dimension in
// chunks of RT_CB blocks of 32 values, double-buffered in LDS.  Each chunk of the tokens' rows and
// the experts' router rows is copied into LDS by global_load_lds_dwordx4 (every wavefront load
// reads whole 128-byte lines) while the previous chunk is computed; the 16-byte chunk q of
// block b sits at position 8 b + (q ^ (b & 7)), so the lanes reading one chunk of their blocks
// hit distinct banks.  Lane (b, token pair) of wavefront w computes the 32-term block sums of
// experts 2w, 2w + 1 against tokens 2p, 2p + 1 (router and token blocks in registers); the block
// sums go to LDS.
//
// The pairwise tree of reduce.rs, level by level over n values (a pair at each level, an odd
// last value carried up), restricted to an aligned run of 2^m values is the same tree over that
// run alone: at level L, value i covers [i 2^L, (i + 1) 2^L) clipped to n, and the run's
// boundaries are multiples of 2^L.  So each of a pair's 8 threads folds its own run of the block
// sums in registers, and one thread folds the 8 run results.
constexpr int RT_T = 4, RT_E = 8, RT_PAIRS = RT_T * RT_E, RT_CB = 32;
constexpr int RT_ROW = RT_CB * 128;                    // bytes of one row's chunk: 4 KB
constexpr int RT_STAGE = (RT_T + RT_E) * RT_ROW;       // 48 KB; two stages
constexpr int RT_MAXB = 256;                           // blocks per row: hidden <= 8192

SYN_DEV float4 rt_chunk(const uint8_t* row, int b, int q) {
    return *reinterpret_cast<const float4*>(row + 16 * (8 * b + (q ^ (b & 7))));
}

// The pairwise tree over v[0..n) (n <= N), in place; the result in v[0].
template <int N>
SYN_DEV float tree_fold(float (&v)[N], int n) {
#pragma unroll
    for (int len = N; len > 1; len = (len + 1) >> 1) {
        // one level for every n in (len / 2, len]: the level's n is len' = min(n, len)
        const int m = n < len ? n : len;
#pragma unroll
        for (int i = 0; i < (len + 1) / 2; ++i)
            if (i < (m + 1) / 2) v[i] = (2 * i + 1 < m) ? v[2 * i] + v[2 * i + 1] : v[2 * i];
        n = (m + 1) / 2;
    }
    return v[0];
}

// Wavefront w issues, for chunk c0, row i of the stage (tokens 0-3, then experts 0-7), blocks
// 8w .. 8w + 7: one 16-byte load a lane (token rows not 16-byte aligned: four 4-byte loads).
template <bool X16>
SYN_DEV void rt_issue(const float* x, const float* router, int rows, int hidden, int n_experts,
                      int t0, int e0, int c0, int nblk, int wave, int lane, uint8_t* stage) {
#pragma unroll
    for (int r = 0; r < RT_T + RT_E; ++r) {
        const uint32_t dst = lds_addr(stage + r * RT_ROW + 1024 * wave);
        const float* base;
        if (r < RT_T) {
            const int t = t0 + r < rows ? t0 + r : rows - 1;
            base = x + (int64_t)t * hidden;
        } else {
            const int e = e0 + r - RT_T < n_experts ? e0 + r - RT_T : n_experts - 1;
            base = router + (int64_t)e * hidden;
        }
        if (X16 || r >= RT_T) {
            const int bq = 64 * wave + lane, bl = bq >> 3, q = (bq & 7) ^ (bl & 7);
            const int b = c0 + bl < nblk ? c0 + bl : nblk - 1;  // past the row: a valid block, unused
            lds_dma16((uint32_t)(b * 128 + 16 * q), base, dst);
        } else {
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int bq = 64 * wave + 16 * s4 + (lane >> 2), bl = bq >> 3, q = (bq & 7) ^ (bl & 7);
                const int b = c0 + bl < nblk ? c0 + bl : nblk - 1;
                lds_dma4((uint32_t)(b * 128 + 16 * q + 4 * (lane & 3)), base, dst + 256 * s4);
            }
        }
    }
}

template <bool X16>  // token rows 16-byte aligned (else they are copied 4 bytes a lane)
__global__ __launch_bounds__(256) void k_moe_logits(const float* __restrict__ router,
                                                    const float* __restrict__ x, int rows,
                                                    int hidden, int n_experts,
                                                    float* __restrict__ logits,
                                                    const uint32_t* __restrict__ active) {
    constexpr int LOADS = X16 ? RT_T + RT_E : 4 * RT_T + RT_E;  // loads per chunk per wavefront
    extern __shared__ __attribute__((aligned(16))) uint8_t rt_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * RT_T, e0 = blockIdx.y * RT_E;
    rows = active_rows(active, 0, rows);
    if (t0 >= rows) return;  // uniform: tokens past the step's active rows
    const int nblk = hidden / 32;
    float* S0 = reinterpret_cast<float*>(rt_lds + 2 * RT_STAGE);  // [RT_PAIRS][nblk]
    rt_issue<X16>(x, router, rows, hidden, n_experts, t0, e0, 0, nblk, wave, lane, rt_lds);
    const int bl = lane & 31, tp = lane >> 5;
    for (int c0 = 0, cur = 0; c0 < nblk; c0 += RT_CB, cur ^= 1) {
        if (c0 + RT_CB < nblk) {
            rt_issue<X16>(x, router, rows, hidden, n_experts, t0, e0, c0 + RT_CB, nblk, wave, lane,
                          rt_lds + (cur ^ 1) * RT_STAGE);
            wait_vm<LOADS>();
        } else {
            wait_vm<0>();
        }
        lds_barrier();
        const uint8_t* st = rt_lds + cur * RT_STAGE;
        const int b = c0 + bl;
        if (b < nblk) {
            float xv[2][32], wv[2][32];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 f = rt_chunk(st + (2 * tp + j) * RT_ROW, bl, q);
                    const float4 g = rt_chunk(st + (RT_T + 2 * wave + j) * RT_ROW, bl, q);
                    xv[j][4 * q] = f.x;
                    xv[j][4 * q + 1] = f.y;
                    xv[j][4 * q + 2] = f.z;
                    xv[j][4 * q + 3] = f.w;
                    wv[j][4 * q] = g.x;
                    wv[j][4 * q + 1] = g.y;
                    wv[j][4 * q + 2] = g.z;
                    wv[j][4 * q + 3] = g.w;
                }
#pragma unroll
            for (int je = 0; je < 2; ++je)
#pragma unroll
                for (int jt = 0; jt < 2; ++jt) {
                    float acc = 0.0f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) acc = acc + wv[je][i] * xv[jt][i];
                    S0[((2 * tp + jt) * RT_E + 2 * wave + je) * nblk + b] = acc;
                }
        }
        lds_barrier();  // this stage is refilled two chunks on
    }
    // the tree: pair pr = tid / 8; thread sub = tid % 8 folds blocks [sub * cs, sub * cs + cs)
    const int pr = tid >> 3, sub = tid & 7;
    int cs = 1;
    while (cs * 8 < nblk) cs <<= 1;  // <= 32
    const int start = sub * cs;
    const int cnt = nblk - start < 0 ? 0 : (nblk - start < cs ? nblk - start : cs);
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = i < cnt ? S0[pr * nblk + start + i] : 0.0f;
    const float run = tree_fold<32>(v, cnt);
    float r8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r8[i] = __shfl(run, (lane & ~7) + i);
    const int nrun = (nblk + cs - 1) / cs;
    const float total = tree_fold<8>(r8, nrun);
    if (sub == 0) {
        const int t = pr / RT_E, e = pr - t * RT_E;
        if (t0 + t < rows && e0 + e < n_experts) logits[(int64_t)(t0 + t) * n_experts + e0 + e] = total;
    }
}

// Logits at many tokens: one workgroup per 32 tokens x 16 experts, two (token, expert) pairs per
// thread (tokens 2g and 2g + 1 against one expert), so each router value a thread reads serves
// two tokens: a wavefront's lanes read 8 token rows and 16 router rows (LDS broadcasts), 12
// distinct 16-byte chunks per pair and step against 20 at one pair a thread.  The rows stream
// through LDS in chunks of 4 blocks (512 bytes a row, padded by 16 bytes so the 16 router rows of
// a read fall in distinct banks), double-buffered by DMA.  Each thread sums each pair's 32-term
// blocks in order and keeps its pairwise tree as a binary stack: block j's sum merges with the
// completed subtrees left of it (level L when bit L of j is set, left + right), and at the end
// the subtrees of the set bits of nblk fold from the smallest up (left + right).  That is
// reduce.rs's level-by-level tree with the odd value carried: the tree over n values is the tree
// over the first 2^m (the largest power of two below n) plus the tree over the rest.
constexpr int LT_T = 32, LT_E = 16, LT_CB = 4;
constexpr int LT_ROW = LT_CB * 128 + 16;          // a row's chunk in LDS: 528 bytes
constexpr int LT_NR = LT_T + LT_E;                // rows a stage holds
constexpr int LT_STAGE = LT_NR * LT_ROW;          // 25,344 bytes
constexpr int LT_NS = 3;                           // ring stages: two chunks in flight
constexpr int LT_CPW = LT_NR / 4;                 // copies per wavefront per chunk: one row each
constexpr int LT_LEVELS = 9;                      // nblk <= 256

// one pair's block sum pushed onto its tree stack (block j, in block order)
SYN_DEV void lt_push(float (&st)[LT_LEVELS], float v, int j) {
    bool carry = true;
#pragma unroll
    for (int L = 0; L < LT_LEVELS; ++L) {
        if (carry) {
            if ((j >> L) & 1) {
                v = st[L] + v;
            } else {
                st[L] = v;
                carry = false;
            }
        }
    }
}
SYN_DEV float lt_total(const float (&st)[LT_LEVELS], int nblk) {
    float total = 0.0f;
    bool have = false;
#pragma unroll
    for (int L = 0; L < LT_LEVELS; ++L) {
        if ((nblk >> L) & 1) {
            total = have ? st[L] + total : st[L];
            have = true;
        }
    }
    return total;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_moe_logits_tile(const float* __restrict__ router,
                                                         const float* __restrict__ x, int rows, int hidden,
                                                         int n_experts, float* __restrict__ logits,
                                                         const uint32_t* __restrict__ active) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lt_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * LT_T, e0 = blockIdx.y * LT_E;
    rows = active_rows(active, 0, rows);
    if (t0 >= rows) return;  // uniform: tokens past the step's active rows
    const int nblk = hidden / 32;
    // wavefront w copies stage rows 12w .. 12w + 11 (tokens 0-31, then experts 0-15): lane l < 32
    // the 16 bytes l of the row's chunk, one copy per row
    auto issue = [&](int c0, uint8_t* stage) {
        const int nb = nblk - c0 < LT_CB ? nblk - c0 : LT_CB;
#pragma unroll
        for (int i = 0; i < LT_CPW; ++i) {
            const int r = LT_CPW * wave + i;
            const float* base;
            if (r < LT_T) {
                const int t = t0 + r < rows ? t0 + r : rows - 1;
                base = x + (int64_t)t * hidden;
            } else {
                const int e = e0 + r - LT_T < n_experts ? e0 + r - LT_T : n_experts - 1;
                base = router + (int64_t)e * hidden;
            }
            if (lane < 8 * nb) lds_dma16(16u * (uint32_t)lane + 128u * (uint32_t)c0, base, lds_addr(stage + r * LT_ROW));
        }
    };
    const int tg = 4 * wave + (lane >> 4), ee = lane & 15;  // tokens 2 tg, 2 tg + 1; expert ee
    float st0[LT_LEVELS], st1[LT_LEVELS];
#pragma unroll
    for (int L = 0; L < LT_LEVELS; ++L) st0[L] = st1[L] = 0.0f;
    issue(0, lt_lds);
    if (LT_CB < nblk) issue(LT_CB, lt_lds + LT_STAGE);
    for (int c0 = 0, cur = 0; c0 < nblk; c0 += LT_CB, cur = cur == LT_NS - 1 ? 0 : cur + 1) {
        if (c0 + LT_CB < nblk)
            wait_vm<LT_CPW>();  // this wavefront's copies of the current chunk, older than the next's
        else
            wait_vm<0>();
        lds_barrier();  // everyone's copies of this chunk landed, and the chunk before is read out
        if (c0 + 2 * LT_CB < nblk)  // into the slot of the chunk before
            issue(c0 + 2 * LT_CB, lt_lds + (cur == 0 ? LT_NS - 1 : cur - 1) * LT_STAGE);
        const uint8_t* stage = lt_lds + cur * LT_STAGE;
        const float4* xr0 = reinterpret_cast<const float4*>(stage + (2 * tg) * LT_ROW);
        const float4* xr1 = reinterpret_cast<const float4*>(stage + (2 * tg + 1) * LT_ROW);
        const float4* wr = reinterpret_cast<const float4*>(stage + (LT_T + ee) * LT_ROW);
        const int nb = nblk - c0 < LT_CB ? nblk - c0 : LT_CB;
        // the chunk's block sums (independent chains), pushed in block order
        float acc0[LT_CB], acc1[LT_CB];
#pragma unroll
        for (int u = 0; u < LT_CB; ++u) acc0[u] = acc1[u] = 0.0f;
#pragma unroll 2
        for (int q = 0; q < 8; ++q) {
#pragma unroll
            for (int u = 0; u < LT_CB; ++u) {
                const int bb = u < nb ? u : 0;  // past the chunk: a valid block, unused
                const float4 wv = wr[8 * bb + q], xa = xr0[8 * bb + q], xb = xr1[8 * bb + q];
                acc0[u] = acc0[u] + wv.x * xa.x;
                acc0[u] = acc0[u] + wv.y * xa.y;
                acc0[u] = acc0[u] + wv.z * xa.z;
                acc0[u] = acc0[u] + wv.w * xa.w;
                acc1[u] = acc1[u] + wv.x * xb.x;
                acc1[u] = acc1[u] + wv.y * xb.y;
                acc1[u] = acc1[u] + wv.z * xb.z;
                acc1[u] = acc1[u] + wv.w * xb.w;
            }
        }
#pragma unroll
        for (int u = 0; u < LT_CB; ++u) {
            if (u < nb) {
                lt_push(st0, acc0[u], c0 + u);
                lt_push(st1, acc1[u], c0 + u);
            }
        }
    }
    const float tot0 = lt_total(st0, nblk), tot1 = lt_total(st1, nblk);
    const int ta = t0 + 2 * tg, tb = ta + 1;
    if (e0 + ee < n_experts) {
        if (ta < rows) logits[(int64_t)ta * n_experts + e0 + ee] = tot0;
        if (tb < rows) logits[(int64_t)tb * n_experts + e0 + ee] = tot1;
    }
}

// The many-token logits kernel from this many rows on (fewer: too few workgroups to fill the
// chip); it copies 16-byte chunks, so the token rows must be 16-byte aligned.
constexpr int LT_MIN_ROWS = 512;

// Softmax and top-k: one wavefront per token (E <= 256, 4 experts per lane).  The selection
// ranks every expert by (probability descending, index ascending), a NaN after every number
// (the spec's order; with a NaN anywhere in a row every probability is NaN and the ranks are the
// indices, as a first-best scan gives).  The order is that of one 64-bit key per expert:
// (NaN ? 0 : |p| bits + 1) << 8 | (255 - e).  Probabilities are exp(.) / sum, never negative, so
// the magnitude bits order them as the float comparison does.
SYN_DEV uint64_t rank_key(float p, int e) {
    const uint32_t b = __builtin_bit_cast(uint32_t, p) & 0x7FFFFFFFu;
    const uint64_t k = p != p ? 0ull : (uint64_t)b + 1ull;
    return (k << 8) | (uint64_t)(255 - e);
}

template <int NQ>  // experts per lane: E <= 64 NQ
__global__ __launch_bounds__(256) void k_moe_topk(const float* __restrict__ logits, int rows,
                                                  int n_experts, int top_k, int renorm,
                                                  int32_t* __restrict__ ids,
                                                  float* __restrict__ wout,
                                                  float* __restrict__ probs_out,
                                                  const uint32_t* __restrict__ active) {
    rows = active_rows(active, 0, rows);
    __shared__ __attribute__((aligned(16))) float sp[4][256];
    __shared__ __attribute__((aligned(16))) uint64_t keys[4][256];
    __shared__ __attribute__((aligned(16))) float selv[4][32];
    __shared__ int seli[4][32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= rows) return;
    float* lg = sp[wave];
    const float* src = logits + (int64_t)t * n_experts;
    // the row maximum as a first-best scan finds it: logit 0, then any strictly larger one
    float m = -__builtin_inff(), l0 = 0.0f;
    for (int e = lane; e < n_experts; e += 64) {
        const float v = src[e];
        lg[e] = v;
        l0 = e == 0 ? v : l0;
        m = v > m ? v : m;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off);
        m = o > m ? o : m;
    }
    l0 = __shfl(l0, 0);
    if (l0 != l0) m = l0;
    for (int e = lane; e < n_experts; e += 64) lg[e] = ref_exp(lg[e] - m);
    wave_lds_sync();
    // F32Fixed sum of the E exponentials: 32-term blocks in order (one lane each), then the
    // pairwise tree over the block sums in one lane (reduce.rs:30-60)
    const int nbk = (n_experts + 31) >> 5;  // <= 8
    float bsum = 0.0f;
    if (lane < nbk) {
        if (lane * 32 + 32 <= n_experts) {
            float4 q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = reinterpret_cast<const float4*>(lg + lane * 32)[i];
#pragma unroll
            for (int i = 0; i < 8; ++i) bsum = (((bsum + q[i].x) + q[i].y) + q[i].z) + q[i].w;
        } else {
            for (int i = lane * 32; i < n_experts; ++i) bsum = bsum + lg[i];
        }
    }
    float b8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b8[i] = __shfl(bsum, i);
    float total = 0.0f;
    {
        int n = nbk;
        while (n > 1) {
            const int half = (n + 1) >> 1;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < half) b8[i] = (2 * i + 1 < n) ? b8[2 * i] + b8[2 * i + 1] : b8[2 * i];
            n = half;
        }
        total = nbk > 0 ? b8[0] : 0.0f;
    }
    uint64_t* kw = keys[wave];
    float v[NQ];
    uint64_t kv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int e = lane + 64 * q;
        v[q] = e < n_experts ? lg[e] / total : 0.0f;
        kv[q] = rank_key(v[q], e);
        if (e < n_experts) {
            kw[e] = kv[q];
            if (probs_out) probs_out[(int64_t)t * n_experts + e] = v[q];
        }
    }
    // keys past E, up to a multiple of 8, rank after every real one
    const int e8 = (n_experts + 7) & ~7;
    if (lane < e8 - n_experts) kw[n_experts + lane] = 0ull;
    wave_lds_sync();
    // rank of each of the lane's experts: how many keys are larger
    int rk[NQ] = {};
    for (int f = 0; f < e8; f += 8) {
        ulonglong2 u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = reinterpret_cast<const ulonglong2*>(kw + f)[i];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) rk[q] += (u[i].x > kv[q] ? 1 : 0) + (u[i].y > kv[q] ? 1 : 0);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (lane + 64 * q < n_experts && rk[q] < top_k) {
            selv[wave][rk[q]] = v[q];
            seli[wave][rk[q]] = lane + 64 * q;
        }
    }
    wave_lds_sync();
    // the k selected, in rank order from +0 (one block: k <= 32)
    float tsum = 0.0f;
    for (int j = 0; j < top_k; j += 4) {
        const float4 q = *reinterpret_cast<const float4*>(&selv[wave][j]);
        tsum = tsum + q.x;
        if (j + 1 < top_k) tsum = tsum + q.y;
        if (j + 2 < top_k) tsum = tsum + q.z;
        if (j + 3 < top_k) tsum = tsum + q.w;
    }
    if (lane < top_k) {
        const float myw = selv[wave][lane];
        ids[(int64_t)t * top_k + lane] = seli[wave][lane];
        wout[(int64_t)t * top_k + lane] = renorm ? myw / tsum : myw;
    }
}

// Two staging areas and the block sums.
size_t moe_logits_lds(int hidden) { return 2ull * RT_STAGE + (size_t)RT_PAIRS * (hidden / 32) * sizeof(float); }

bool moe_route_supported(int hidden) { return hidden > 0 && hidden % 32 == 0 && hidden / 32 <= RT_MAXB; }

void launch_moe_route(const float* router, const float* x, int rows, int hidden, int n_experts,
                      int top_k, int renorm, int32_t* ids, float* w, float* probs, float* logits,
                      hipStream_t stream, const uint32_t* active) {
    const dim3 grid((rows + RT_T - 1) / RT_T, (n_experts + RT_E - 1) / RT_E);
    const size_t lds = moe_logits_lds(hidden);
    static const hipError_t lds_ok =
        hipFuncSetAttribute((const void*)k_moe_logits<true>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    static const hipError_t lds_ok4 =
        hipFuncSetAttribute((const void*)k_moe_logits<false>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)lds_ok;  // a refusal shows as the launch's error
    (void)lds_ok4;
    if (rows >= LT_MIN_ROWS && ((uintptr_t)x & 15) == 0 && ((uintptr_t)router & 15) == 0) {
        static const hipError_t lt_ok = hipFuncSetAttribute((const void*)k_moe_logits_tile,
                                                            hipFuncAttributeMaxDynamicSharedMemorySize, LT_NS * LT_STAGE);
        (void)lt_ok;  // a refusal shows as the launch's error
        const dim3 lg((rows + LT_T - 1) / LT_T, (n_experts + LT_E - 1) / LT_E);
        hipLaunchKernelGGL(k_moe_logits_tile, lg, dim3(256), LT_NS * LT_STAGE, stream, router, x, rows, hidden, n_experts,
                           logits, active);
    } else if (((uintptr_t)x & 15) == 0)
        hipLaunchKernelGGL(k_moe_logits<true>, grid, dim3(256), lds, stream, router, x, rows, hidden, n_experts, logits,
                           active);
    else
        hipLaunchKernelGGL(k_moe_logits<false>, grid, dim3(256), lds, stream, router, x, rows, hidden, n_experts,
                           logits, active);
    const dim3 tg((rows + 3) / 4);
#define SYN_TOPK(NQ)                                                                                           \
    hipLaunchKernelGGL(k_moe_topk<NQ>, tg, dim3(256), 0, stream, logits, rows, n_experts, top_k, renorm, ids, w, \
                       probs, active)
    if (n_experts <= 64)
        SYN_TOPK(1);
    else if (n_experts <= 128)
        SYN_TOPK(2);
    else if (n_experts <= 192)
        SYN_TOPK(3);
    else
        SYN_TOPK(4);
#undef SYN_TOPK
}

// ============================================================================================
// Packing: counting sort of slots by expert, stable in slot order (moe.rs:431-457)
// ============================================================================================
// err[0]: 1 when an id is out of range, else 0; err[1]: the largest expert's entry count.

constexpr int PACK_BATCH = 8;  // chunks of 64 ids a wavefront loads at once

// One workgroup of 1024 threads; wave w owns the contiguous slot range [w*per, (w+1)*per).
// Pass 1 counts per (wave, expert) in LDS; pass 2 scans to per-(wave, expert) bases; pass 3
// places each wave's slots in order (64 at a time, ranks among equal experts by ballots).
// A route id outside [0, n_experts) sets *err and the layer writes nothing.
__global__ __launch_bounds__(1024) void k_moe_pack(const int32_t* __restrict__ ids, int nslots,
                                                   int n_experts, uint32_t* __restrict__ offsets,
                                                   uint32_t* __restrict__ slots,
                                                   uint32_t* __restrict__ err,
                                                   const uint32_t* __restrict__ active, int top_k,
                                                   const int32_t* __restrict__ site,
                                                   uint32_t* __restrict__ report) {
    if (active) nslots = active_rows(active, 0, nslots / top_k) * top_k;  // the active rows' slots
    // Every id is checked; a slot whose expert the site mask leaves out is neither counted nor
    // packed, so no later kernel computes or writes it.
    extern __shared__ uint32_t cnt[];  // [16][n_experts]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (nslots + 15) / 16;
    const int s_begin = wave * per;
    const int s_end = s_begin + per < nslots ? s_begin + per : nslots;
    for (int i = tid; i < 16 * n_experts; i += 1024) cnt[i] = 0;
    __shared__ uint32_t bad;  // the first slot whose id names no expert, or ~0
    if (tid == 0) bad = ~0u;
    __syncthreads();
    // the wave's ids PACK_BATCH chunks of 64 at a time, their loads in flight together
    for (int c0 = s_begin; c0 < s_end; c0 += 64 * PACK_BATCH) {
        int ev[PACK_BATCH];
#pragma unroll
        for (int u = 0; u < PACK_BATCH; ++u) {
            const int s = c0 + 64 * u + lane;
            ev[u] = s < s_end ? ids[s] : 0;
        }
#pragma unroll
        for (int u = 0; u < PACK_BATCH; ++u) {
            const int s = c0 + 64 * u + lane;
            if (s >= s_end) continue;
            const int e = ev[u];
            if (e < 0 || e >= n_experts)
                atomicMin(&bad, (uint32_t)s);
            else if (!site || site[e] != 0)
                atomicAdd(&cnt[wave * n_experts + e], 1u);
        }
    }
    __syncthreads();
    if (bad != ~0u) {
        if (tid == 0) {
            *err = 1u;
            // the caller's report words (host memory the host reads after the stream): the
            // first failing launch since the host last cleared word 0 writes 1 + slot, the id
            // and top_k
            if (report) {
                uint32_t none = 0;
                if (__hip_atomic_compare_exchange_strong(report, &none, bad + 1u, __ATOMIC_RELAXED,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)) {
                    __hip_atomic_store(report + 1, (uint32_t)ids[bad], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    __hip_atomic_store(report + 2, (uint32_t)top_k, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
                }
            }
        }
        return;
    }
    // scan, expert-major then wave-minor: per-expert totals, an exclusive scan of the totals in
    // one wavefront (4 experts a lane), then each expert's per-wave bases.
    __shared__ uint32_t tot[256];
    __shared__ uint32_t base_e[257];
    for (int e = tid; e < n_experts; e += 1024) {
        uint32_t c = 0;
        for (int w = 0; w < 16; ++w) c += cnt[w * n_experts + e];
        tot[e] = c;
    }
    __syncthreads();
    if (wave == 0) {
        uint32_t v[4], run = 0, most = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = lane * 4 + q;
            v[q] = e < n_experts ? tot[e] : 0u;
            most = v[q] > most ? v[q] : most;
            run += v[q];
        }
        uint32_t incl = run;  // inclusive scan of the lane totals
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(incl, off);
            if (lane >= off) incl += o;
        }
        uint32_t ex = incl - run;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = lane * 4 + q;
            if (e < n_experts) base_e[e] = ex;
            ex += v[q];
        }
        if (lane == 63) base_e[n_experts] = incl;  // the total
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t o = __shfl_xor(most, off);
            most = o > most ? o : most;
        }
        if (lane == 0) {
            err[0] = 0u;
            err[1] = most;  // the largest expert's entry count, which sizes the FFN item space
        }
    }
    __syncthreads();
    for (int e = tid; e <= n_experts; e += 1024) offsets[e] = base_e[e];
    for (int e = tid; e < n_experts; e += 1024) {
        uint32_t run = base_e[e];
        for (int w = 0; w < 16; ++w) {
            const uint32_t c = cnt[w * n_experts + e];
            cnt[w * n_experts + e] = run;
            run += c;
        }
    }
    __syncthreads();
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int ev[PACK_BATCH];
    for (int c0 = s_begin; c0 < s_end; c0 += 64) {
        const int u = ((c0 - s_begin) >> 6) % PACK_BATCH;  // uniform
        if (u == 0)  // the next PACK_BATCH chunks' ids, loaded together
#pragma unroll
            for (int v = 0; v < PACK_BATCH; ++v) {
                const int sv = c0 + 64 * v + lane;
                ev[v] = sv < s_end ? ids[sv] : -1;
            }
        const int s = c0 + lane;
        int e = -1;
#pragma unroll
        for (int v = 0; v < PACK_BATCH; ++v) e = v == u ? ev[v] : e;
        const bool live = e >= 0 && (!site || site[e] != 0);
        // lanes holding the same expert
        uint64_t same = __ballot(live);
#pragma unroll
        for (int bit = 0; bit < 9; ++bit) {
            const bool b = (e >> bit) & 1;
            const uint64_t m = __ballot(live && b);
            same &= b ? m : ~m;
        }
        if (live) {
            const uint32_t rank = (uint32_t)__popcll(same & lt);
            const uint32_t base = cnt[wave * n_experts + e];
            slots[base + rank] = (uint32_t)s;
        }
        // advance this wave's cursors: the highest lane of each expert group adds the count
        const bool last = live && ((same >> lane) == 1ull);
        wave_lds_sync();
        if (last) cnt[wave * n_experts + e] += (uint32_t)__popcll(same);
        wave_lds_sync();
    }
}

void launch_moe_pack(const int32_t* ids, int nslots, int n_experts, uint32_t* offsets,
                     uint32_t* slots, uint32_t* err, hipStream_t stream, const uint32_t* active, int top_k,
                     const int32_t* site, uint32_t* report) {
    hipLaunchKernelGGL(k_moe_pack, dim3(1), dim3(1024), sizeof(uint32_t) * 16 * n_experts, stream,
                       ids, nslots, n_experts, offsets, slots, err, active, top_k, site, report);
}

// ============================================================================================
// Gather + Q8_K: entry i (packed order) takes row slots[i] / top_k of x
// ============================================================================================

size_t moe_act_bytes(int64_t nentries, int k) {
    const int64_t nb = k / 256;
    // scale rows padded to 4 entries, 64 bytes past the end: the expert kernels read 16-byte
    // aligned windows of scales
    return align_up((size_t)(nentries * k), 256) +
           align_up((size_t)(align_up((size_t)nentries, 4) * nb * 4 + 64), 256) +
           align_up((size_t)(nentries * nb * 16), 256);
}
MoeAct moe_act_at(uint8_t* base, int64_t nentries, int k) {
    const int64_t nb = k / 256;
    MoeAct a;
    a.codes = (int8_t*)base;
    a.d = (float*)(base + align_up((size_t)(nentries * k), 256));
    a.dstride = (int)align_up((size_t)nentries, 4);
    a.lh = (uint8_t*)a.d + align_up((size_t)(a.dstride * nb * 4 + 64), 256);
    a.nentries = (int)nentries;
    return a;
}

// One wavefront per (entry, 256-value block).  Lane l quantizes values 4l..4l+3: sub-block
// j = l/8, k part p = (l%8)/2, bytes 4(l%2)..+3 of that part, stored at
// 64p + 16(j%4) + 8(j/4): the two sub-blocks j and j + 4 that one expert-kernel lane multiplies
// sit side by side.
__global__ __launch_bounds__(256) void k_moe_gather_q8k(const float* __restrict__ x,
                                                        const uint32_t* __restrict__ slots,
                                                        int nentries, int top_k, int k,
                                                        const uint32_t* __restrict__ err,
                                                        MoeAct a, int gather,
                                                        const uint32_t* __restrict__ total) {
    if (err && err[0]) return;
    if (total) nentries = (int)(*total < (uint32_t)nentries ? *total : (uint32_t)nentries);  // packed entries
    const int nb = k / 256;
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (int64_t)nentries * nb) return;
    const int i = (int)(item / nb), b = (int)(item - (int64_t)i * nb);
    const int64_t src_row = gather ? (int64_t)(slots[i] / (uint32_t)top_k) : i;
    const Q8KLane r = q8k_block_lane(x + src_row * k + (int64_t)b * 256, lane);
    const int j = lane >> 3, p = (lane & 7) >> 1;
    *reinterpret_cast<uint32_t*>(a.codes + (int64_t)i * k + (int64_t)b * 256 + 64 * p +
                                 16 * (j & 3) + 8 * (j >> 2) + 4 * (lane & 1)) = r.packed;
    uint8_t* lh = a.lh + ((int64_t)i * nb + b) * 16;
    if ((lane & 7) == 0) {
        lh[j] = (uint8_t)(r.sum32 & 127);
        lh[8 + j] = (uint8_t)(r.sum32 >> 7);
    }
    if (lane == 0) a.d[(int64_t)b * a.dstride + i] = r.d;
}

void launch_moe_gather_q8k(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                           const uint32_t* err, MoeAct a, int gather, hipStream_t stream, const uint32_t* total) {
    const int64_t items = (int64_t)nentries * (k / 256);
    if (items == 0) return;
    hipLaunchKernelGGL(k_moe_gather_q8k, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, x,
                       slots, nentries, top_k, k, err, a, gather, total);
}

// ============================================================================================
// TILE64 repack of Q4_K rows (whole 64-row runs of nb super-blocks): one thread per 16-byte chunk
// ============================================================================================

__global__ __launch_bounds__(256) void k_tile64_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       uint64_t chunks, int nb, int inverse) {
    const uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const uint64_t blk = c / 9;  // the block in GGUF order: row blk / nb, super-block blk % nb
    const uint32_t q = (uint32_t)(c - blk * 9);
    const uint64_t row = blk / (uint64_t)nb, b = blk - row * (uint64_t)nb;
    const uint64_t at = (row / TILE64_ROWS) * TILE64_ROWS * (uint64_t)nb + b * TILE64_ROWS + row % TILE64_ROWS;
    const uint64_t g_off = blk * 144 + 16 * q, t_off = at * 144 + 16 * q;
    const uint64_t from = inverse ? t_off : g_off, to = inverse ? g_off : t_off;
    *reinterpret_cast<uint4*>(dst + to) = *reinterpret_cast<const uint4*>(src + from);
}

void launch_tile64_repack(const uint8_t* src, uint8_t* dst, uint64_t bytes, int k, int inverse, hipStream_t stream) {
    const uint64_t chunks = bytes / 16;
    if (chunks == 0) return;
    hipLaunchKernelGGL(k_tile64_repack, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, src, dst, chunks,
                       k / 256, inverse);
}

// ============================================================================================
// Grouped Q4_K product on the int8 matrix cores
// ============================================================================================
//
// A workgroup item is (expert, 64 consecutive weight rows, up to 16 consecutive entries of the
// expert); each of its four wavefronts takes 16 of the rows and walks their super-blocks in
// order.  The workgroup streams every super-block's operands - the 64 rows of each weight
// matrix and the entries' codes, sums and scales - from global memory straight into LDS
// (global_load_lds_dwordx4, no registers held while the loads fly), two super-blocks ahead of
// the arithmetic, in a ring of three stages.
//
// The entries go four at a time (decode routes a few entries to each expert).  A product
// v_mfma_i32_16x16x32_i8 has 16 A rows; row 4j' + t carries entry t's codes of sub-block
// 4h + j' (zero in the other three products of the group), so four accumulating products
// (sub-blocks 4h..4h+3) leave lane l = 16p + c holding the exact I32 sums D_h[t] of weight row c
// and sub-block 4h + p against entries t = 0..3.  The lane scales them, s[t] = sc_p D_0[t] +
// sc_{4+p} D_1[t]; summing s over the four lanes of the row (two lane swaps) gives S1 of entry
// p, and S2 = sum_j m_j s_j of entry p comes from its packed sub-block sums with sdot4.  The
// lane then folds the super-block term of (row c, entry p) into its accumulator
// (gemv.rs:539-547).

// The shape of one expert kernel: NM weight matrices, WV wavefronts of 16 rows each, up to CH
// entries (CH / 4 groups) per item.  One stage in LDS: NM weight tiles [16 WV rows][144 bytes],
// the entries' codes [CH][256] (16-byte chunk q of entry t at position q ^ (t & 3): a 16-byte
// LDS read serves four lanes of each quarter-wave per pass, here entries c & 3 times chunks
// 4p + jq, whose positions then differ), their sums [CH][16], then the
// 16-byte-aligned window of CH + 4 scales holding theirs.
template <int NM_, int WV_, int CH_>
struct MoeCfg {
    static constexpr int NM = NM_, WV = WV_, CH = CH_, NG = CH_ / 4;
    static constexpr int THREADS = 64 * WV;
    static constexpr int ROWS = 16 * WV;
    static constexpr int W = ROWS * 144;
    static constexpr int WCHUNKS = NM * ROWS * 9;        // 16-byte chunks of the weight tiles
    static constexpr int WSLOTS = (WCHUNKS + 63) / 64;
    static constexpr int CODES = NM * W;
    static constexpr int LH = CODES + CH * 256;
    static constexpr int DX = LH + CH * 16;
    static constexpr int BYTES = DX + (CH / 4 + 1) * 16;
    static constexpr int SLOTS = WSLOTS + NG + 1;         // wavefront loads per stage
    static constexpr int PER_WAVE = (SLOTS + WV - 1) / WV;  // each wavefront issues as many
    static_assert(CH % 4 == 0 && CH <= 16 && CH + CH / 4 + 1 <= 64, "entry chunk");
};
constexpr int MOE_STAGES = 3;

// One wavefront's load slot of a stage: the lane's global address of super-block 0 and its
// step per super-block, whether the lane loads, and the slot's LDS offset inside the stage.
// Every load is 16 bytes; lane L of a slot writes LDS offset + 16 L.
struct Slot {
    const uint8_t* src;
    uint32_t step;
    bool on;    // this lane loads
    bool live;  // the slot loads at all (uniform): not padding, not an absent entry group
    int lds;
    // weights in the X8 layout (a dense matrix): the lane's chunk q of super-block g0 + b, at
    // x8_chunk_offset from the matrix base `src`, over a matrix of xnb super-blocks
    bool x8;
    int xq;
    uint64_t xg0, xnb;
};

// The weight rows of an item: its first row (row0, or its byte offset in GGUF order) and, for a
// dense matrix, the last row (later rows are clamped to it) and the X8 layout.
struct ItemRows {
    int row0, row_max;
    uint32_t row0_off;
    bool x8;
    uint64_t nblocks;  // super-blocks of the whole matrix (X8)
    bool tiled = false;  // TILE64: block b of the item's 64 rows is one piece (row0 a multiple of 64)
};

template <class C>
SYN_DEV Slot make_slot(int s, const uint8_t* const (&bases)[C::NM], const ItemRows& ir, uint32_t rb,
                       const MoeAct& a, int k, int ent0, int nent) {
    const int lane = threadIdx.x & 63;
    Slot r;
    r.on = true;
    r.live = s < C::SLOTS;
    r.x8 = false;
    r.xq = 0;
    r.xg0 = r.xnb = 0;
    if (s >= C::SLOTS) s = C::SLOTS - 1;
    if (s < C::WSLOTS) {
        // chunk ci = 64 s + lane of the tiles: matrix ci / (9 ROWS), then row, then part of 9
        const int ci0 = 64 * s + lane;
        r.on = ci0 < C::WCHUNKS;
        const int ci = r.on ? ci0 : 0;
        const int m = ci / (9 * C::ROWS), rem = ci - m * (9 * C::ROWS);
        const int rr = rem / 9, q = rem % 9;
        if (ir.x8) {
            const int row = ir.row0 + rr < ir.row_max ? ir.row0 + rr : ir.row_max;
            r.x8 = true;
            r.xq = q;
            r.xg0 = (uint64_t)row * (uint64_t)(k / 256);
            r.xnb = ir.nblocks;
            r.src = bases[m];
        } else {
            const uint32_t rrc = ir.row_max >= 0 && ir.row0 + rr > ir.row_max ? (uint32_t)(ir.row_max - ir.row0) : (uint32_t)rr;
            r.src = bases[m] + (ir.row0_off + rrc * (ir.tiled ? 144u : rb) + 16u * (uint32_t)q);
        }
        r.step = ir.tiled ? (uint32_t)C::ROWS * 144u : 144u;
        r.lds = s * 1024;
    } else if (s < C::WSLOTS + C::NG) {
        // entries 4j..4j+3: position q of entry t holds its chunk q ^ (t & 3)
        const int j = s - C::WSLOTS, t = 4 * j + (lane >> 4), q = lane & 15;
        r.live = r.live && 4 * j < nent;
        const int ec = ent0 + (t < nent ? t : nent - 1);
        r.src = (const uint8_t*)a.codes + ((uint32_t)ec * (uint32_t)k + 16u * (uint32_t)(q ^ (t & 3)));
        r.step = 256u;
        r.lds = C::CODES + j * 1024;
    } else if (lane < C::CH) {
        // sums of entry `lane`
        const int ec = ent0 + (lane < nent ? lane : nent - 1);
        r.src = a.lh + (uint32_t)ec * (uint32_t)(k / 256) * 16u;
        r.step = 16u;
        r.lds = C::LH;
    } else {
        // the next lanes: the scales from ent0 rounded down to 4 (rows padded to 4 entries)
        const int w = lane - C::CH;
        r.on = w <= C::CH / 4;
        r.src = (const uint8_t*)(a.d + (ent0 & ~3) + 4 * (r.on ? w : 0));
        r.step = 4u * (uint32_t)a.dstride;
        r.lds = C::LH;
    }
    return r;
}

// The load is written as assembly so the compiler does not track it: it would otherwise wait
// for every load into LDS still in flight before each LDS read, the next stages' included.
// The explicit waits of the ring order the stages instead.
SYN_DEV void issue_slot(const Slot& sl, int b, uint8_t* stage) {
    if (sl.live && sl.on) {
        const uint8_t* src = sl.x8 ? sl.src + x8_chunk_offset(sl.xg0 + (uint32_t)b, sl.xq, sl.xnb)
                                   : sl.src + (uint64_t)sl.step * (uint32_t)b;
        const uint32_t dst = (uint32_t)(uintptr_t)(lds_ptr)(stage + sl.lds);
        // the LDS address is an m0 operand (the compiler sets m0; s_nop is the wait state)
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :
                     : "v"(src), "{m0}"(dst)
                     : "memory");
    }
}

SYN_DEV long pack2(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// One super-block of 16 weight rows of NM matrices, as lane (c, p) holds it: row c's 16-byte
// header and its codes at 16 + 32 g + 8 p (g = 0..3).
template <int NM>
struct WBlock {
    v4u hdr[NM];
    uint32_t q[NM][8];
};

// The super-block's arithmetic against the item's entry groups: the entries' codes [CH][256]
// (chunk-swizzled), their sums [CH][16] and the scale window `dxw`, all in LDS.  acc[m][g]
// (row c, entry 4g + p) accumulates the super-block's term (gemv.rs:539-547).
template <int NM, int NG>
SYN_DEV void q4k_block(const WBlock<NM>& w, const uint8_t* codes, const uint8_t* lhs, const float* dxw, int ent0,
                       int ngroups, float (&acc)[NM][NG]) {
    const int lane = threadIdx.x & 63, c = lane & 15, p = lane >> 4, jq = c >> 2;
    long bq[NM][8];  // B operands: the row's codes of sub-block j, k part p
    uint32_t mns[NM][2];
    int sc0[NM], sc1[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t lo = w.q[m][2 * (j >> 1)], hi = w.q[m][2 * (j >> 1) + 1];
            const uint32_t c0 = (j & 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
            const uint32_t c1 = (j & 1) ? (hi >> 4) & 0x0F0F0F0Fu : hi & 0x0F0F0F0Fu;
            bq[m][j] = pack2(c0, c1);
        }
        // get_scale_min_k4 (gemv.rs:528-537) on packed bytes: scales of sub-blocks p and 4 + p,
        // mins of sub-blocks 0-3 | 4-7
        const uint32_t w0 = w.hdr[m].y, w1 = w.hdr[m].z, w2 = w.hdr[m].w;
        const uint32_t sc_lo = w0 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (w2 & 0x0F0F0F0Fu) | ((w0 >> 2) & 0x30303030u);
        sc0[m] = (int)((sc_lo >> (8 * p)) & 0xFFu);
        sc1[m] = (int)((sc_hi >> (8 * p)) & 0xFFu);
        mns[m][0] = w1 & 0x3F3F3F3Fu;
        mns[m][1] = ((w2 >> 4) & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    }
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        if (g >= ngroups) break;  // uniform
        // entry 4g + (c & 3): its codes of sub-blocks jq and jq + 4, k part p
        const int ta = 4 * g + (c & 3);
        const v4u ap = *reinterpret_cast<const v4u*>(codes + ta * 256 + 16 * ((4 * p + jq) ^ (c & 3)));
        const int to = 4 * g + p;  // the lane's output entry
        const v4u lh = *reinterpret_cast<const v4u*>(lhs + 16 * to);
        const float dx = dxw[(ent0 & 3) + to];
        v4i d0[NM], d1[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) d0[m] = d1[m] = z;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const long a0 = jj == jq ? pack2(ap.x, ap.y) : 0;
            const long a1 = jj == jq ? pack2(ap.z, ap.w) : 0;
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                d0[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bq[m][jj], d0[m], 0, 0, 0);
                d1[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bq[m][4 + jj], d1[m], 0, 0, 0);
            }
        }
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            // |D| <= 32 * 15 * 127 fits 24 bits: v_mad_i32_i24
            int sv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) sv[t] = sc0[m] * ((d0[m][t] << 8) >> 8) + sc1[m] * ((d1[m][t] << 8) >> 8);
            // sum over the row's four lanes, entry p left in lane p: rows p, p^1 exchange two
            // values (odd rows' first <-> even rows' second), then lane halves one
            const auto r0 = __builtin_amdgcn_permlane16_swap(sv[0], sv[1], false, false);
            const auto r1 = __builtin_amdgcn_permlane16_swap(sv[2], sv[3], false, false);
            const int z0 = (int)r0[0] + (int)r0[1], z1 = (int)r1[0] + (int)r1[1];
            const auto r2 = __builtin_amdgcn_permlane32_swap(z0, z1, false, false);
            const int s1 = (int)r2[0] + (int)r2[1];
            const int s2 = sdot4(mns[m][0], lh.x, sdot4(mns[m][1], lh.y, 0)) +
                           128 * sdot4(mns[m][0], lh.z, sdot4(mns[m][1], lh.w, 0));
            const float d = f16_to_f32(w.hdr[m].x), dmin = f16_to_f32(w.hdr[m].x >> 16);
            acc[m][g] = acc[m][g] + ((d * dx) * (float)s1 - (dmin * dx) * (float)s2);
        }
    }
}

// One super-block of the wavefront's 16 rows of NM matrices from the stage's weight tiles.
template <class C>
SYN_DEV void q4k_super(const uint8_t* st, int wave, int ent0, int ngroups, float (&acc)[C::NM][C::NG]) {
    const int lane = threadIdx.x & 63, c = lane & 15, p = lane >> 4;
    WBlock<C::NM> w;
#pragma unroll
    for (int m = 0; m < C::NM; ++m) {
        const uint8_t* row = st + m * C::W + (16 * wave + c) * 144;
        w.hdr[m] = *reinterpret_cast<const v4u*>(row);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint2 v = *reinterpret_cast<const uint2*>(row + 16 + 32 * g + 8 * p);
            w.q[m][2 * g] = v.x;
            w.q[m][2 * g + 1] = v.y;
        }
    }
    q4k_block<C::NM, C::NG>(w, st + C::CODES, st + C::LH, reinterpret_cast<const float*>(st + C::DX), ent0,
                            ngroups, acc);
}

// The item's super-blocks in order through an NS-stage LDS ring (three for the MoE layer).
// Each wavefront issues the same loads for every stage (the entry groups the item has); before
// the arithmetic on super-block b it waits until only the loads of b + 1 .. b + NS - 2 may still
// fly, then the barrier makes the stage whole for the workgroup.
template <class C, int NS = MOE_STAGES>
SYN_DEV void ffn_rows(const uint8_t* const (&bases)[C::NM], const ItemRows& ir, uint32_t rb,
                      const MoeAct& a, int k, int ent0, int nent, int wave, uint8_t* lds,
                      float (&acc)[C::NM][C::NG]) {
    const int nb = k / 256;
    const int ngroups = (nent + 3) >> 2;
    Slot sl[C::PER_WAVE];
    int live = 0;  // loads this wavefront issues per stage
#pragma unroll
    for (int i = 0; i < C::PER_WAVE; ++i) {
        sl[i] = make_slot<C>(wave + C::WV * i, bases, ir, rb, a, k, ent0, nent);
        live += sl[i].live ? 1 : 0;
    }
#pragma unroll
    for (int q = 0; q < NS - 1; ++q)
        if (q < nb)
#pragma unroll
            for (int i = 0; i < C::PER_WAVE; ++i) issue_slot(sl[i], q, lds + q * C::BYTES);
#pragma unroll 1
    for (int b = 0; b < nb; ++b) {
        const int ahead = nb - 1 - b < NS - 2 ? nb - 1 - b : NS - 2;
        wait_vm_n<C::PER_WAVE * (NS - 2)>(ahead * live);
        lds_barrier();
        const int bn = b + NS - 1;
        if (bn < nb) {
#pragma unroll
            for (int i = 0; i < C::PER_WAVE; ++i) issue_slot(sl[i], bn, lds + (bn % NS) * C::BYTES);
        }
        q4k_super<C>(lds + (b % NS) * C::BYTES, wave, ent0, ngroups, acc);
    }
}

// Entry range of expert e's items: offsets[e]..offsets[e+1].
struct MoeItems {
    const uint32_t* offsets;
    int n_experts;
    int row_groups;  // weight rows / rows per item
    int chunk;       // entries per item
    // dense > 0: one matrix (n_experts 1, no offsets) whose entries are its first `dense` rows of
    // activations, or *active of them when `active` is set (a step descriptor's rows_active)
    int dense;
    const uint32_t* active;
};

SYN_DEV int moe_dense_rows(const MoeItems& it) {
    if (!it.active) return it.dense;
    const uint32_t a = *it.active;
    return a < (uint32_t)it.dense ? (int)a : it.dense;
}

// Maps a flat item index to (expert, row group, entry chunk); items of an expert with fewer
// entries are empty.  Items: expert-major, then entry chunk, then row group.  The item space,
// n_experts * row_groups * max_chunks, is sized on the device from the largest expert.
SYN_DEV int moe_max_chunks(const MoeItems& it, const uint32_t* err) {
    const int most = it.dense ? moe_dense_rows(it) : (int)err[1];
    return (most + it.chunk - 1) / it.chunk;
}
SYN_DEV bool moe_item(const MoeItems& it, int item, int max_chunks, int& e, int& rg, int& ent0,
                      int& nent) {
    const int per_e = it.row_groups * max_chunks;
    e = item / per_e;
    const int r = item - e * per_e;
    const int ch = r / it.row_groups;
    rg = r - ch * it.row_groups;
    if (e >= it.n_experts) return false;
    const int b0 = it.dense ? 0 : (int)it.offsets[e], b1 = it.dense ? moe_dense_rows(it) : (int)it.offsets[e + 1];
    ent0 = b0 + ch * it.chunk;
    if (ent0 >= b1) return false;
    nent = b1 - ent0 < it.chunk ? b1 - ent0 : it.chunk;
    return true;
}

// gate/up + SiLU: h[entry][row] = silu(gate_row . x) * (up_row . x) (moe.rs:466-499).
template <int WV, int CH>
__global__ __launch_bounds__(64 * WV) void k_moe_gateup(const uint8_t* __restrict__ gate,
                                                        const uint8_t* __restrict__ up, int inter,
                                                        int hidden, MoeItems it, MoeAct a,
                                                        const uint32_t* __restrict__ err,
                                                        float* __restrict__ h, int tiled) {
    using C = MoeCfg<2, WV, CH>;
    static_assert(C::ROWS == TILE64_ROWS, "an item's rows are one TILE64 run");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if (err[0]) return;
    const int max_chunks = moe_max_chunks(it, err);
    const int total = it.n_experts * it.row_groups * max_chunks;
    const int lane = threadIdx.x & 63, p = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rb = (uint32_t)(hidden / 256) * 144u;
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        int e, rg, ent0, nent;
        if (!moe_item(it, item, max_chunks, e, rg, ent0, nent)) continue;  // uniform per workgroup
        const int64_t ebytes = (int64_t)inter * rb;
        const uint8_t* const bases[2] = {gate + e * ebytes, up + e * ebytes};
        float acc[2][C::NG] = {};
        ItemRows ir{rg * C::ROWS, -1, (uint32_t)(rg * C::ROWS) * rb, false, 0};
        ir.tiled = tiled != 0;
        ffn_rows<C>(bases, ir, rb, a, hidden, ent0, nent, wave, lds, acc);
        const int row = rg * C::ROWS + wave * 16 + (lane & 15);
#pragma unroll
        for (int g = 0; g < C::NG; ++g)
            if (4 * g + p < nent)
                h[(int64_t)(ent0 + 4 * g + p) * inter + row] = ref_silu(acc[0][g]) * acc[1][g];
        lds_barrier();  // the ring is refilled by the next item
    }
}

// down: out[slot][row] = down_row . hq[entry], written to the entry's slot (the reference's
// scatter, moe.rs:501-515); the experts in GGUF order or, with 64-row items, TILE64 (`layout`).
// With it.dense (a dense Gemv of a few rows): one matrix `down` of `hidden` rows (GGUF order, or
// X8), out[entry][row], no slots and no error word.
template <int WV, int CH, int NS = MOE_STAGES>
__global__ __launch_bounds__(64 * WV) void k_moe_down(const uint8_t* __restrict__ down, int hidden,
                                                      int inter, MoeItems it, MoeAct a,
                                                      const uint32_t* __restrict__ slots,
                                                      const uint32_t* __restrict__ err,
                                                      float* __restrict__ out, int layout) {
    using C = MoeCfg<1, WV, CH>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if (err && err[0]) return;
    const int max_chunks = moe_max_chunks(it, err);
    const int total = it.n_experts * it.row_groups * max_chunks;
    const int lane = threadIdx.x & 63, p = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rb = (uint32_t)(inter / 256) * 144u;
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        int e, rg, ent0, nent;
        if (!moe_item(it, item, max_chunks, e, rg, ent0, nent)) continue;  // uniform per workgroup
        const uint8_t* const bases[1] = {down + e * ((int64_t)hidden * rb)};
        float acc[1][C::NG] = {};
        ItemRows ir{rg * C::ROWS, it.dense ? hidden - 1 : -1, (uint32_t)(rg * C::ROWS) * rb, layout == LAYOUT_X8,
                    (uint64_t)hidden * (uint64_t)(inter / 256)};
        ir.tiled = layout == LAYOUT_TILE64;
        ffn_rows<C, NS>(bases, ir, rb, a, inter, ent0, nent, wave, lds, acc);
        const int row = rg * C::ROWS + wave * 16 + (lane & 15);
#pragma unroll
        for (int g = 0; g < C::NG; ++g) {
            const int ent = ent0 + 4 * g + p;
            if (4 * g + p < nent && row < hidden) out[(int64_t)(slots ? (int)slots[ent] : ent) * hidden + row] = acc[0][g];
        }
        lds_barrier();  // the ring is refilled by the next item
    }
}

// The grid covers every item of the common case (the largest expert within one entry chunk)
// with one workgroup each; larger item spaces, sized on the device, are walked grid-stride.
static unsigned moe_grid(const MoeItems& it, int nentries) {
    int64_t items = (int64_t)it.n_experts * it.row_groups;
    const int64_t cap = (int64_t)it.n_experts * it.row_groups * ((nentries + it.chunk - 1) / it.chunk);
    items = items < cap ? items : cap;
    return (unsigned)(items > 0 ? items : 1);
}

// gate/up: four wavefronts (64 rows), up to 16 entries per item; down: four wavefronts, up to
// 12 entries per item: its three stages of 12.4 KB leave room for four workgroups per CU (three
// at 16 entries), which made the 64-token decode layer 2-3 % faster; an expert of 13 to 24
// entries then streams its down rows twice
constexpr int GU_WV = 4, GU_CH = 16;
constexpr int DN_WV = 4, DN_CH = 12;

void launch_moe_gateup(const uint8_t* gate, const uint8_t* up, int n_experts, int hidden,
                       int inter, const uint32_t* offsets, int nentries, MoeAct a,
                       const uint32_t* err, float* h, hipStream_t stream, int layout) {
    using C = MoeCfg<2, GU_WV, GU_CH>;
    const MoeItems it{offsets, n_experts, inter / C::ROWS, C::CH, 0, nullptr};
    const int lds = MOE_STAGES * C::BYTES;
    static const hipError_t lds_ok = hipFuncSetAttribute(
        (const void*)k_moe_gateup<GU_WV, GU_CH>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)lds_ok;  // a refusal shows as the launch's error
    hipLaunchKernelGGL((k_moe_gateup<GU_WV, GU_CH>), dim3(moe_grid(it, nentries)), dim3(C::THREADS),
                       lds, stream, gate, up, inter, hidden, it, a, err, h, layout == LAYOUT_TILE64 ? 1 : 0);
}

void launch_moe_down(const uint8_t* down, int n_experts, int hidden, int inter,
                     const uint32_t* offsets, int nentries, MoeAct a, const uint32_t* slots,
                     const uint32_t* err, float* out, hipStream_t stream, int layout) {
    using C = MoeCfg<1, DN_WV, DN_CH>;
    static_assert(C::ROWS == TILE64_ROWS, "an item's rows are one TILE64 run");
    const MoeItems it{offsets, n_experts, hidden / C::ROWS, C::CH, 0, nullptr};
    const int lds = MOE_STAGES * C::BYTES;
    static const hipError_t lds_ok = hipFuncSetAttribute(
        (const void*)k_moe_down<DN_WV, DN_CH>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)lds_ok;  // a refusal shows as the launch's error
    hipLaunchKernelGGL((k_moe_down<DN_WV, DN_CH>), dim3(moe_grid(it, nentries)), dim3(C::THREADS),
                       lds, stream, down, hidden, inter, it, a, slots, err, out,
                       layout == LAYOUT_TILE64 ? (int)LAYOUT_TILE64 : (int)LAYOUT_SOURCE);
}

// A dense Q4_K Gemv of 2 to 31 rows on the decode expert kernel: the matrix as one expert, the
// rows as its entries (quantized by launch_moe_gather_q8k without a gather), y[row][out].
// Narrow matrices take 16-row items so that the grid still covers the GPU.
// The dense form's ring: three stages, as the MoE layer's (eight measured no faster: the
// launch's fixed cost and the rows' read pattern bound it, not the loads in flight).
constexpr int DENSE_STAGES = MOE_STAGES, DENSE_CH = 16;

template <int WV>
static void launch_dense_wv(const uint8_t* W, int x8, int n_out, int k, MoeAct a, int rows, float* y,
                            hipStream_t stream, const uint32_t* active) {
    using C = MoeCfg<1, WV, DENSE_CH>;
    const MoeItems it{nullptr, 1, (n_out + C::ROWS - 1) / C::ROWS, C::CH, rows, active};
    const int lds = DENSE_STAGES * C::BYTES;
    static const hipError_t lds_ok = hipFuncSetAttribute(
        (const void*)k_moe_down<WV, DENSE_CH, DENSE_STAGES>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)lds_ok;  // a refusal shows as the launch's error
    const unsigned grid = (unsigned)it.row_groups * (unsigned)((rows + C::CH - 1) / C::CH);
    hipLaunchKernelGGL((k_moe_down<WV, DENSE_CH, DENSE_STAGES>), dim3(grid), dim3(C::THREADS), lds, stream, W, n_out,
                       k, it, a, nullptr, nullptr, y, x8 ? (int)LAYOUT_X8 : (int)LAYOUT_SOURCE);
}

// The K-split form over one dense matrix (rows of a multiple of 4 super-blocks): a workgroup of
// four wavefronts owns 16 weight rows and up to CH (4, 8 or 16) entries; a stage holds 4
// super-blocks, one per wavefront, each in the one-wavefront expert stage layout (MoeCfg<1, 1,
// CH>: the same copies and the same super-block arithmetic, q4k_super).  The entry chunk is
// sized to the rows, so that small ones leave room in LDS for more workgroups per CU.  A wavefront's term of a super-block
// comes out of q4k_super exactly (its sum starts at -0.0, and -0.0 + t = t); the terms go to LDS
// at [entry][row][4] and, after the next barrier, lane o of the workgroup adds output o's four
// in super-block order.  The fold, and every bit, is the one-wavefront kernel's with four
// wavefronts on the rows.
constexpr int DK_WAVES = 4;

template <int NS, int CH>
__global__ __launch_bounds__(64 * DK_WAVES) void k_q4k_rows_splitk(const uint8_t* __restrict__ W, int n_out, int k,
                                                                   MoeItems it, MoeAct a, float* __restrict__ out,
                                                                   int x8) {
    using C = MoeCfg<1, 1, CH>;
    constexpr int OUTS = 16 * CH;  // outputs of the workgroup: entry o / 16, row o % 16
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int STAGE = DK_WAVES * C::BYTES;
    const int max_chunks = moe_max_chunks(it, nullptr);
    const int lane = threadIdx.x & 63, p = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = k / 256, nst = nb / DK_WAVES;
    const uint32_t rb = (uint32_t)nb * 144u;
    float* terms = reinterpret_cast<float*>(lds + NS * STAGE);  // [2][OUTS][4]
    int e, rg, ent0, nent;
    if (!moe_item(it, (int)blockIdx.x, max_chunks, e, rg, ent0, nent)) return;  // uniform per workgroup
    const uint8_t* const bases[1] = {W};
    const ItemRows ir{rg * 16, n_out - 1, (uint32_t)(rg * 16) * rb, x8 != 0, (uint64_t)n_out * (uint64_t)nb};
    const int ngroups = (nent + 3) >> 2;
    // every wavefront makes the same slots (its 16 rows, the item's entries) and issues them for
    // its own super-block of each stage into its own part of the stage
    Slot sl[C::PER_WAVE];
    int live = 0;
#pragma unroll
    for (int i = 0; i < C::PER_WAVE; ++i) {
        sl[i] = make_slot<C>(i, bases, ir, rb, a, k, ent0, nent);
        live += sl[i].live ? 1 : 0;
    }
    auto issue = [&](int s) {
        uint8_t* part = lds + (s % NS) * STAGE + wave * C::BYTES;
#pragma unroll
        for (int i = 0; i < C::PER_WAVE; ++i) issue_slot(sl[i], DK_WAVES * s + wave, part);
    };
    const int o = (int)threadIdx.x;  // the output this lane folds (o < OUTS)
    float acc = 0.0f;
    auto fold = [&](int buf) {
        if (o < OUTS) {
            const float4 v = *reinterpret_cast<const float4*>(terms + buf * OUTS * 4 + o * 4);
            acc = (((acc + v.x) + v.y) + v.z) + v.w;
        }
    };
#pragma unroll
    for (int q = 0; q < NS - 1; ++q)
        if (q < nst) issue(q);
#pragma unroll 1
    for (int s = 0; s < nst; ++s) {
        const int ahead = nst - 1 - s < NS - 2 ? nst - 1 - s : NS - 2;
        wait_vm_n<C::PER_WAVE * (NS - 2)>(ahead * live);
        lds_barrier();  // stage s whole; stage s - 1 and the terms of s - 2 read out
        if (s > 0) fold((s - 1) & 1);
        if (s + NS - 1 < nst) issue(s + NS - 1);
        float t[1][C::NG];
#pragma unroll
        for (int g = 0; g < C::NG; ++g) t[0][g] = -0.0f;
        q4k_super<C>(lds + (s % NS) * STAGE + wave * C::BYTES, 0, ent0, ngroups, t);
        float* tw = terms + (s & 1) * OUTS * 4;
#pragma unroll
        for (int g = 0; g < C::NG; ++g)
            if (g < ngroups) tw[((4 * g + p) * 16 + c) * 4 + wave] = t[0][g];
    }
    lds_barrier();
    fold((nst - 1) & 1);
    const int ent = o >> 4, row = rg * 16 + (o & 15);
    if (o < OUTS && ent < nent && row < n_out) out[(int64_t)(ent0 + ent) * n_out + row] = acc;
}

template <int NS, int CH>
static void launch_dense_splitk(const uint8_t* W, int x8, int n_out, int k, MoeAct a, int rows, float* y,
                                hipStream_t stream, const uint32_t* active) {
    using C = MoeCfg<1, 1, CH>;
    const MoeItems it{nullptr, 1, (n_out + 15) / 16, C::CH, rows, active};
    const int lds = NS * DK_WAVES * C::BYTES + 2 * 16 * CH * 4 * 4;
    static const hipError_t lds_ok = hipFuncSetAttribute((const void*)k_q4k_rows_splitk<NS, CH>,
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)lds_ok;  // a refusal shows as the launch's error
    const unsigned grid = (unsigned)it.row_groups * (unsigned)((rows + C::CH - 1) / C::CH);
    hipLaunchKernelGGL((k_q4k_rows_splitk<NS, CH>), dim3(grid), dim3(64 * DK_WAVES), lds, stream, W, n_out, k, it, a,
                       y, x8);
}

// The K-split form over X8 rows (rows of a multiple of 8 super-blocks, each row whole runs):
// eight wavefronts on 16 weight rows, a stage holding one run (super-blocks 8s..8s+7) of every
// row.  The weights are copied along whole 128-byte lines (eight consecutive lanes read one
// line: chunk q of the run's eight super-blocks) into a shared region in line order, 16-byte
// chunks [row][q][i ^ ((row >> 1) & 7)] (the XOR spreads 16 rows' reads of one super-block over
// distinct banks), and wavefront i reads super-block i of the run from it; each wavefront copies
// its own super-block's entries (codes, sums, scales) as the expert stage does.  The arithmetic
// (q4k_block), the terms and their fold in super-block order are the four-wavefront form's.
constexpr int X8R_WV = 8;
constexpr int X8R_WBYTES = 16 * 9 * 128;  // one run of 16 rows
constexpr int X8R_WSLOTS = X8R_WBYTES / 1024;

template <class C>
constexpr int x8r_entry_bytes() { return C::BYTES - C::CODES; }  // codes, sums, scale window
template <class C>
constexpr int x8r_stage() { return X8R_WBYTES + X8R_WV * x8r_entry_bytes<C>(); }

// Super-block i of the run, as lane (c, p) holds it, from the line-order region: row c's header is
// chunk 0, its codes at 16 + 32 g + 8 p are chunk 1 + 2 g + p / 2 at 8 (p & 1).
SYN_DEV WBlock<1> x8r_block(const uint8_t* wl, int i) {
    const int lane = threadIdx.x & 63, c = lane & 15, p = lane >> 4;
    const uint8_t* r = wl + c * (9 * 128) + 16 * (i ^ ((c >> 1) & 7));
    WBlock<1> w;
    w.hdr[0] = *reinterpret_cast<const v4u*>(r);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint2 v = *reinterpret_cast<const uint2*>(r + (1 + 2 * g + (p >> 1)) * 128 + 8 * (p & 1));
        w.q[0][2 * g] = v.x;
        w.q[0][2 * g + 1] = v.y;
    }
    return w;
}

template <int NS, int CH>
__global__ __launch_bounds__(64 * X8R_WV) void k_q4k_rows_x8(const uint8_t* __restrict__ W, int n_out, int k,
                                                              MoeItems it, MoeAct a, float* __restrict__ out) {
    using C = MoeCfg<1, 1, CH>;
    constexpr int WV = X8R_WV, OUTS = 16 * CH, EB = x8r_entry_bytes<C>(), STAGE = x8r_stage<C>();
    constexpr int WPER = (X8R_WSLOTS + WV - 1) / WV;  // weight slots per wavefront (at most)
    constexpr int EPER = C::SLOTS - C::WSLOTS;         // entry slots per wavefront
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int max_chunks = moe_max_chunks(it, nullptr);
    const int lane = threadIdx.x & 63, p = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = k / 256, nst = nb / 8;
    const uint32_t rb = (uint32_t)nb * 144u;
    float* terms = reinterpret_cast<float*>(lds + NS * STAGE);  // [2][OUTS][WV]
    int e, rg, ent0, nent;
    if (!moe_item(it, (int)blockIdx.x, max_chunks, e, rg, ent0, nent)) return;  // uniform per workgroup
    const int ngroups = (nent + 3) >> 2;
    // weight slots: chunk ci = 64 slot + lane is line ci / 8 (row r = ci / 72, chunk q of the run)
    // at position ci % 8, which holds super-block (ci % 8) ^ ((r >> 1) & 7) of the run; rows past
    // the matrix read its last row (their outputs are not written)
    Slot ws[WPER];
    int live = 0;
#pragma unroll
    for (int u = 0; u < WPER; ++u) {
        const int slot = wave + WV * u;
        const int ci = 64 * (slot < X8R_WSLOTS ? slot : 0) + lane;
        const int line = ci >> 3, r = line / 9, q = line - 9 * r;
        const int row = rg * 16 + r < n_out ? rg * 16 + r : n_out - 1;
        ws[u].src = W + ((uint64_t)row * rb + 128u * (uint32_t)q + 16u * (uint32_t)((ci & 7) ^ ((r >> 1) & 7)));
        ws[u].step = 1152u;  // one run
        ws[u].on = true;
        ws[u].live = slot < X8R_WSLOTS;
        ws[u].x8 = false;
        ws[u].xq = 0;
        ws[u].xg0 = ws[u].xnb = 0;
        ws[u].lds = slot * 1024;
        live += ws[u].live ? 1 : 0;
    }
    // this wavefront's entry slots for its super-block of each run
    const uint8_t* const bases[1] = {W};
    const ItemRows ir{rg * 16, n_out - 1, 0u, false, 0};
    Slot es[EPER];
#pragma unroll
    for (int i = 0; i < EPER; ++i) {
        es[i] = make_slot<C>(C::WSLOTS + i, bases, ir, rb, a, k, ent0, nent);
        live += es[i].live ? 1 : 0;
    }
    auto issue = [&](int s) {
        uint8_t* st = lds + (s % NS) * STAGE;
#pragma unroll
        for (int u = 0; u < WPER; ++u) issue_slot(ws[u], s, st);
        // make_slot's entry offsets start at C::CODES: shift them to this wavefront's part
        uint8_t* part = st + X8R_WBYTES + wave * EB - C::CODES;
#pragma unroll
        for (int i = 0; i < EPER; ++i) issue_slot(es[i], 8 * s + wave, part);
    };
    const int o = (int)threadIdx.x;  // the output this lane folds (o < OUTS)
    float acc = 0.0f;
    auto fold = [&](int buf) {
        if (o < OUTS) {
#pragma unroll
            for (int h = 0; h < WV / 4; ++h) {
                const float4 v = *reinterpret_cast<const float4*>(terms + (buf * OUTS + o) * WV + 4 * h);
                acc = (((acc + v.x) + v.y) + v.z) + v.w;
            }
        }
    };
#pragma unroll
    for (int q = 0; q < NS - 1; ++q)
        if (q < nst) issue(q);
#pragma unroll 1
    for (int s = 0; s < nst; ++s) {
        const int ahead = nst - 1 - s < NS - 2 ? nst - 1 - s : NS - 2;
        wait_vm_n<(WPER + EPER) * (NS - 2)>(ahead * live);
        lds_barrier();  // stage s whole; stage s - 1 and the terms of s - 2 read out
        if (s > 0) fold((s - 1) & 1);
        if (s + NS - 1 < nst) issue(s + NS - 1);
        const uint8_t* st = lds + (s % NS) * STAGE;
        const uint8_t* part = st + X8R_WBYTES + wave * EB;
        float t[1][C::NG];
#pragma unroll
        for (int g = 0; g < C::NG; ++g) t[0][g] = -0.0f;
        const WBlock<1> w = x8r_block(st, wave);
        q4k_block<1, C::NG>(w, part, part + (C::LH - C::CODES), reinterpret_cast<const float*>(part + (C::DX - C::CODES)),
                            ent0, ngroups, t);
        float* tw = terms + (s & 1) * OUTS * WV;
#pragma unroll
        for (int g = 0; g < C::NG; ++g)
            if (g < ngroups) tw[((4 * g + p) * 16 + c) * WV + wave] = t[0][g];
    }
    lds_barrier();
    fold((nst - 1) & 1);
    const int ent = o >> 4, row = rg * 16 + (o & 15);
    if (o < OUTS && ent < nent && row < n_out) out[(int64_t)(ent0 + ent) * n_out + row] = acc;
}

template <int NS, int CH>
static void launch_rows_x8(const uint8_t* W, int n_out, int k, MoeAct a, int rows, float* y, hipStream_t stream,
                           const uint32_t* active) {
    using C = MoeCfg<1, 1, CH>;
    const MoeItems it{nullptr, 1, (n_out + 15) / 16, C::CH, rows, active};
    const int lds = NS * x8r_stage<C>() + 2 * 16 * CH * X8R_WV * 4;
    static const hipError_t lds_ok = hipFuncSetAttribute((const void*)k_q4k_rows_x8<NS, CH>,
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)lds_ok;  // a refusal shows as the launch's error
    const unsigned grid = (unsigned)it.row_groups * (unsigned)((rows + C::CH - 1) / C::CH);
    hipLaunchKernelGGL((k_q4k_rows_x8<NS, CH>), dim3(grid), dim3(64 * X8R_WV), lds, stream, W, n_out, k, it, a, y);
}

void launch_q4k_dense_rows(const uint8_t* W, int x8, int n_out, int k, MoeAct a, int rows, float* y,
                           hipStream_t stream, const uint32_t* active) {
    const int nb = k / 256;
    if (x8 && nb % 8 == 0) {  // X8 rows of whole runs: the line-order form
        if (rows <= 4)
            launch_rows_x8<2, 4>(W, n_out, k, a, rows, y, stream, active);
        else if (rows <= 8)
            launch_rows_x8<2, 8>(W, n_out, k, a, rows, y, stream, active);
        else
            launch_rows_x8<2, 16>(W, n_out, k, a, rows, y, stream, active);
    } else if (nb % DK_WAVES == 0) {
        if (rows <= 4)
            launch_dense_splitk<2, 4>(W, x8, n_out, k, a, rows, y, stream, active);
        else if (rows <= 8)
            launch_dense_splitk<2, 8>(W, x8, n_out, k, a, rows, y, stream, active);
        else
            launch_dense_splitk<2, 16>(W, x8, n_out, k, a, rows, y, stream, active);
    } else if (n_out >= 8192) {
        launch_dense_wv<2>(W, x8, n_out, k, a, rows, y, stream, active);
    } else {
        launch_dense_wv<1>(W, x8, n_out, k, a, rows, y, stream, active);
    }
}

// ============================================================================================
// MoeCombine (moe/tests.rs:541-556)
// ============================================================================================

// One workgroup per (row, 1024 columns).  The row's ids and weights go to LDS, each slot's rank
// in (expert id, slot) order (a stable sort by id) is counted by its own thread, then each
// thread adds its four columns over the slots in that order (float4 loads where the rows are
// 16-byte aligned).
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ out,
                                                     const int32_t* __restrict__ ids,
                                                     const float* __restrict__ w, int top_k,
                                                     int hidden, int vec, float* __restrict__ y,
                                                     const uint32_t* __restrict__ active) {
    __shared__ int order[64];
    __shared__ int sid[64];
    __shared__ float sw[64];
    const int r = blockIdx.y, tid = threadIdx.x;
    if (r >= active_rows(active, 0, (int)gridDim.y)) return;  // uniform: a row past the active ones
    if (tid < top_k) {
        sid[tid] = ids[(int64_t)r * top_k + tid];
        sw[tid] = w[(int64_t)r * top_k + tid];
    }
    __syncthreads();
    if (tid < top_k) {
        const int v = sid[tid];
        int rank = 0;
        for (int i = 0; i < top_k; ++i) {
            const int u = sid[i];
            rank += (u < v || (u == v && i < tid)) ? 1 : 0;
        }
        order[rank] = tid;
    }
    __syncthreads();
    const int c = blockIdx.x * 1024 + 4 * tid;
    if (c >= hidden) return;
    const float* base = out + (int64_t)r * top_k * hidden;
    if (vec) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int a2 = 0; a2 < top_k; ++a2) {
            const int j = order[a2];
            const float wj = sw[j];
            const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)j * hidden + c);
            acc.x = acc.x + wj * v.x;
            acc.y = acc.y + wj * v.y;
            acc.z = acc.z + wj * v.z;
            acc.w = acc.w + wj * v.w;
        }
        *reinterpret_cast<float4*>(y + (int64_t)r * hidden + c) = acc;
    } else {
        const int n = hidden - c < 4 ? hidden - c : 4;
        for (int q = 0; q < n; ++q) {
            float acc = 0.0f;
            for (int a2 = 0; a2 < top_k; ++a2) {
                const int j = order[a2];
                acc = acc + sw[j] * base[(int64_t)j * hidden + c + q];
            }
            y[(int64_t)r * hidden + c + q] = acc;
        }
    }
}

void launch_moe_combine(const float* out, const int32_t* ids, const float* w, int rows, int top_k,
                        int hidden, float* y, hipStream_t stream, const uint32_t* active) {
    if (rows == 0 || hidden == 0) return;
    const int vec = hidden % 4 == 0 && (reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((hidden + 1023) / 1024), (unsigned)rows),
                       dim3(256), 0, stream, out, ids, w, top_k, hidden, vec, y, active);
}

// MoeCombine as the IR binds it (crates/kernels/src/op/kind.rs:244, crates/graph/src/ir/
// signature.rs:153): per row, the routed slots in rank order (slot j is rank j; the binding carries
// no expert ids), then the shared experts' outputs in input order, y = 0.0, y += w_j * v_j, y +=
// shared_s, in F32 without fused multiply-add.  One workgroup per (row, 1024 columns), four
// columns a thread.
__global__ __launch_bounds__(256) void k_moe_combine_ranked(const float* __restrict__ out,
                                                            const float* __restrict__ w, SharedOuts sh,
                                                            int top_k, int hidden, int vec,
                                                            float* __restrict__ y,
                                                            const uint32_t* __restrict__ active) {
    __shared__ float sw[64];
    const int r = blockIdx.y, tid = threadIdx.x;
    if (r >= active_rows(active, 0, (int)gridDim.y)) return;  // uniform: a row past the active ones
    if (tid < top_k) sw[tid] = w[(int64_t)r * top_k + tid];
    __syncthreads();
    const int c = blockIdx.x * 1024 + 4 * tid;
    if (c >= hidden) return;
    const float* base = out + (int64_t)r * top_k * hidden;
    if (vec) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int j = 0; j < top_k; ++j) {
            const float wj = sw[j];
            const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)j * hidden + c);
            acc.x = acc.x + wj * v.x;
            acc.y = acc.y + wj * v.y;
            acc.z = acc.z + wj * v.z;
            acc.w = acc.w + wj * v.w;
        }
        for (int s2 = 0; s2 < sh.n; ++s2) {
            const float4 v = *reinterpret_cast<const float4*>(sh.p[s2] + (int64_t)r * hidden + c);
            acc.x = acc.x + v.x;
            acc.y = acc.y + v.y;
            acc.z = acc.z + v.z;
            acc.w = acc.w + v.w;
        }
        *reinterpret_cast<float4*>(y + (int64_t)r * hidden + c) = acc;
    } else {
        const int n = hidden - c < 4 ? hidden - c : 4;
        for (int q = 0; q < n; ++q) {
            float acc = 0.0f;
            for (int j = 0; j < top_k; ++j) acc = acc + sw[j] * base[(int64_t)j * hidden + c + q];
            for (int s2 = 0; s2 < sh.n; ++s2) acc = acc + sh.p[s2][(int64_t)r * hidden + c + q];
            y[(int64_t)r * hidden + c + q] = acc;
        }
    }
}

void launch_moe_combine_ranked(const float* out, const float* w, const SharedOuts& sh, int rows, int top_k,
                               int hidden, float* y, hipStream_t stream, const uint32_t* active) {
    if (rows == 0 || hidden == 0) return;
    uintptr_t align = reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(y);
    for (int i = 0; i < sh.n; ++i) align |= reinterpret_cast<uintptr_t>(sh.p[i]);
    const int vec = hidden % 4 == 0 && align % 16 == 0;
    hipLaunchKernelGGL(k_moe_combine_ranked, dim3((unsigned)((hidden + 1023) / 1024), (unsigned)rows),
                       dim3(256), 0, stream, out, w, sh, top_k, hidden, vec, y, active);
}

}  // namespace syn
