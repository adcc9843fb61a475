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

// Logits: one workgroup per (TT tokens, EC experts).  The block sums of the chunk go to LDS,
// then the pairwise tree runs level by level in LDS (ping-pong), exactly as reduce.rs defines.
// EC (at most 32) is sized so the tokens' rows and the sums fit 64 KB of LDS.

template <int TT>
__global__ __launch_bounds__(256) void k_moe_logits(const float* __restrict__ router,
                                                    const float* __restrict__ x, int rows,
                                                    int hidden, int n_experts, int EC,
                                                    float* __restrict__ logits) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * TT;
    const int e0 = blockIdx.y * EC;
    const int ec = n_experts - e0 < EC ? n_experts - e0 : EC;
    const int nblk = hidden / 32;
    float* xs = sm;                              // [TT][hidden]
    float* S0 = xs + TT * hidden;  // [TT][EC][nblk]
    float* S1 = S0 + TT * EC * nblk;  // [TT][EC][nblk]
    for (int i = tid; i < TT * hidden; i += 256) {
        const int t = i / hidden, c = i - t * hidden;
        xs[i] = (t0 + t < rows) ? x[(int64_t)(t0 + t) * hidden + c] : 0.0f;
    }
    __syncthreads();
    for (int p = tid; p < ec * nblk; p += 256) {
        const int e = p / nblk, b = p - e * nblk;
        const float4* wr = reinterpret_cast<const float4*>(router + (int64_t)(e0 + e) * hidden + b * 32);
        float wv[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 f = wr[q];
            wv[4 * q] = f.x;
            wv[4 * q + 1] = f.y;
            wv[4 * q + 2] = f.z;
            wv[4 * q + 3] = f.w;
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const float* xb = xs + t * hidden + b * 32;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) acc = acc + wv[i] * xb[i];
            S0[(t * EC + e) * nblk + b] = acc;
        }
    }
    __syncthreads();
    float* src = S0;
    float* dst = S1;
    for (int n = nblk; n > 1; n = (n + 1) >> 1) {
        const int half = (n + 1) >> 1;
        for (int p = tid; p < TT * ec * half; p += 256) {
            const int te = p / half, i = p - te * half;
            const int t = te / ec, e = te - t * ec;
            const float* sp = src + (t * EC + e) * nblk;
            dst[(t * EC + e) * nblk + i] = (2 * i + 1 < n) ? sp[2 * i] + sp[2 * i + 1] : sp[2 * i];
        }
        __syncthreads();
        float* tmp = src;
        src = dst;
        dst = tmp;
    }
    for (int p = tid; p < TT * ec; p += 256) {
        const int t = p / ec, e = p - t * ec;
        if (t0 + t < rows) logits[(int64_t)(t0 + t) * n_experts + e0 + e] = src[(t * EC + e) * nblk];
    }
}

// Softmax and top-k: one wavefront per token (E <= 256, 4 experts per lane).
__global__ __launch_bounds__(256) void k_moe_topk(const float* __restrict__ logits, int rows,
                                                  int n_experts, int top_k, int renorm,
                                                  int32_t* __restrict__ ids,
                                                  float* __restrict__ wout,
                                                  float* __restrict__ probs_out) {
    __shared__ float sp[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= rows) return;
    float* lg = sp[wave];
    const float* src = logits + (int64_t)t * n_experts;
    float m = -__builtin_inff();
    for (int e = lane; e < n_experts; e += 64) {
        lg[e] = src[e];
        m = lg[e] > m ? lg[e] : m;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off);
        m = o > m ? o : m;
    }
    for (int e = lane; e < n_experts; e += 64) lg[e] = ref_exp(lg[e] - m);
    wave_lds_sync();
    // F32Fixed sum of the E exponentials: 32-term blocks in order (one lane each), then the
    // pairwise tree over the block sums in one lane (reduce.rs:30-60)
    const int nbk = (n_experts + 31) >> 5;  // <= 8
    float bsum = 0.0f;
    if (lane < nbk) {
        const int s1 = n_experts < lane * 32 + 32 ? n_experts : lane * 32 + 32;
        for (int i = lane * 32; i < s1; ++i) bsum = bsum + lg[i];
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
    for (int e = lane; e < n_experts; e += 64) lg[e] = lg[e] / total;
    wave_lds_sync();
    if (probs_out)
        for (int e = lane; e < n_experts; e += 64) probs_out[(int64_t)t * n_experts + e] = lg[e];
    // top-k: k rounds of (probability desc, index asc) over the lane's experts
    float v[4];
    int vi[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = lane + 64 * q;
        v[q] = e < n_experts ? lg[e] : 0.0f;
        vi[q] = e < n_experts ? e : 0x7FFFFFFF;
    }
    float tsum = 0.0f;
    float myw = 0.0f;
    int myid = 0;
    for (int j = 0; j < top_k; ++j) {
        float bv = 0.0f;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (vi[q] != 0x7FFFFFFF && (bi == 0x7FFFFFFF || v[q] > bv)) {
                bv = v[q];
                bi = vi[q];
            }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (vi[q] == bi) vi[q] = 0x7FFFFFFF;  // taken
        tsum = tsum + bv;  // the k selected, in rank order from +0 (one block: k <= 32)
        if (lane == j) {
            myw = bv;
            myid = bi;
        }
    }
    if (lane < top_k) {
        ids[(int64_t)t * top_k + lane] = myid;
        wout[(int64_t)t * top_k + lane] = renorm ? myw / tsum : myw;
    }
}

constexpr size_t ROUTE_LDS = 64 * 1024;

// Experts per workgroup for TT tokens of `hidden` values: up to 32, as many as fit the LDS.
int moe_logits_ec(int tt, int hidden) {
    const int64_t rest = (int64_t)ROUTE_LDS - 4ll * tt * hidden;
    const int64_t ec = rest > 0 ? rest / (8ll * tt * (hidden / 32)) : 0;
    return (int)(ec < 32 ? ec : 32);
}
size_t moe_logits_lds(int tt, int hidden, int ec) {
    return sizeof(float) * ((size_t)tt * hidden + 2ull * tt * ec * (hidden / 32));
}

bool moe_route_supported(int hidden) { return moe_logits_ec(1, hidden) >= 1; }

void launch_moe_route(const float* router, const float* x, int rows, int hidden, int n_experts,
                      int top_k, int renorm, int32_t* ids, float* w, float* probs, float* logits,
                      hipStream_t stream) {
    // Two tokens per workgroup share each router block once there are enough tokens and a
    // full chunk of experts still fits.
    const int ec2 = moe_logits_ec(2, hidden);
    if (rows >= 256 && ec2 >= 32) {
        hipLaunchKernelGGL((k_moe_logits<2>), dim3((rows + 1) / 2, (n_experts + ec2 - 1) / ec2),
                           dim3(256), moe_logits_lds(2, hidden, ec2), stream, router, x, rows, hidden,
                           n_experts, ec2, logits);
    } else {
        const int ec = moe_logits_ec(1, hidden);
        hipLaunchKernelGGL((k_moe_logits<1>), dim3(rows, (n_experts + ec - 1) / ec), dim3(256),
                           moe_logits_lds(1, hidden, ec), stream, router, x, rows, hidden, n_experts,
                           ec, logits);
    }
    hipLaunchKernelGGL(k_moe_topk, dim3((rows + 3) / 4), dim3(256), 0, stream, logits, rows,
                       n_experts, top_k, renorm, ids, w, probs);
}

// ============================================================================================
// Packing: counting sort of slots by expert, stable in slot order (moe.rs:431-457)
// ============================================================================================
// err[0]: 1 when an id is out of range, else 0; err[1]: the largest expert's entry count.

// One workgroup of 1024 threads; wave w owns the contiguous slot range [w*per, (w+1)*per).
// Pass 1 counts per (wave, expert) in LDS; pass 2 scans to per-(wave, expert) bases; pass 3
// places each wave's slots in order (64 at a time, ranks among equal experts by ballots).
// A route id outside [0, n_experts) sets *err and the layer writes nothing.
__global__ __launch_bounds__(1024) void k_moe_pack(const int32_t* __restrict__ ids, int nslots,
                                                   int n_experts, uint32_t* __restrict__ offsets,
                                                   uint32_t* __restrict__ slots,
                                                   uint32_t* __restrict__ err) {
    extern __shared__ uint32_t cnt[];  // [16][n_experts]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (nslots + 15) / 16;
    const int s_begin = wave * per;
    const int s_end = s_begin + per < nslots ? s_begin + per : nslots;
    for (int i = tid; i < 16 * n_experts; i += 1024) cnt[i] = 0;
    __shared__ uint32_t bad;
    if (tid == 0) bad = 0;
    __syncthreads();
    for (int s = s_begin + lane; s < s_end; s += 64) {
        const int e = ids[s];
        if (e < 0 || e >= n_experts)
            atomicOr(&bad, 1u);
        else
            atomicAdd(&cnt[wave * n_experts + e], 1u);
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) *err = 1u;
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
    for (int c0 = s_begin; c0 < s_end; c0 += 64) {
        const int s = c0 + lane;
        const bool live = s < s_end;
        const int e = live ? ids[s] : -1;
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
                     uint32_t* slots, uint32_t* err, hipStream_t stream) {
    hipLaunchKernelGGL(k_moe_pack, dim3(1), dim3(1024), sizeof(uint32_t) * 16 * n_experts, stream,
                       ids, nslots, n_experts, offsets, slots, err);
}

// ============================================================================================
// Gather + Q8_K: entry i (packed order) takes row slots[i] / top_k of x
// ============================================================================================

size_t moe_act_bytes(int64_t nentries, int k) {
    const int64_t nb = k / 256;
    // the scales carry 64 bytes of pad: the expert kernels read four entries' scales at once
    return align_up((size_t)(nentries * k), 256) + align_up((size_t)(nentries * nb * 4 + 64), 256) +
           align_up((size_t)(nentries * nb * 16), 256);
}
MoeAct moe_act_at(uint8_t* base, int64_t nentries, int k) {
    const int64_t nb = k / 256;
    MoeAct a;
    a.codes = (int8_t*)base;
    a.d = (float*)(base + align_up((size_t)(nentries * k), 256));
    a.lh = (uint8_t*)a.d + align_up((size_t)(nentries * nb * 4 + 64), 256);
    a.nentries = (int)nentries;
    return a;
}

// One wavefront per (entry, 256-value block).  Lane l quantizes values 4l..4l+3: sub-block
// j = l/8, k part p = (l%8)/2, bytes 4(l%2)..+3 of that part.
__global__ __launch_bounds__(256) void k_moe_gather_q8k(const float* __restrict__ x,
                                                        const uint32_t* __restrict__ slots,
                                                        int nentries, int top_k, int k,
                                                        const uint32_t* __restrict__ err,
                                                        MoeAct a, int gather) {
    if (err[0]) return;
    const int nb = k / 256;
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (int64_t)nentries * nb) return;
    const int i = (int)(item / nb), b = (int)(item - (int64_t)i * nb);
    const int64_t src_row = gather ? (int64_t)(slots[i] / (uint32_t)top_k) : i;
    const Q8KLane r = q8k_block_lane(x + src_row * k + (int64_t)b * 256, lane);
    const int j = lane >> 3, p = (lane & 7) >> 1;
    *reinterpret_cast<uint32_t*>(a.codes + (int64_t)i * k + (int64_t)b * 256 + 64 * p + 8 * j +
                                 4 * (lane & 1)) = r.packed;
    uint8_t* lh = a.lh + ((int64_t)i * nb + b) * 16;
    if ((lane & 7) == 0) {
        lh[j] = (uint8_t)(r.sum32 & 127);
        lh[8 + j] = (uint8_t)(r.sum32 >> 7);
    }
    if (lane == 0) a.d[(int64_t)b * nentries + i] = r.d;
}

void launch_moe_gather_q8k(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                           const uint32_t* err, MoeAct a, int gather, hipStream_t stream) {
    const int64_t items = (int64_t)nentries * (k / 256);
    if (items == 0) return;
    hipLaunchKernelGGL(k_moe_gather_q8k, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, x,
                       slots, nentries, top_k, k, err, a, gather);
}

// ============================================================================================
// Grouped Q4_K product on the int8 matrix cores
// ============================================================================================
//
// A workgroup item is (expert, 64 consecutive weight rows, up to 16 consecutive entries of the
// expert); each of its four wavefronts takes 16 of the rows and walks their super-blocks in
// order with the next super-block's loads in flight.  The entries' codes of a super-block are
// staged once in LDS for the four wavefronts.  Per 32-weight sub-block j, one
// v_mfma_i32_16x16x32_i8: lane l = 16p + c holds weight row c (B operand: the row's 8 codes
// k = 8p..8p+7 of the sub-block) and entry c (A operand: the entry's codes at the same k), and
// receives D[entry 4p+i][row c], i = 0..3: the exact I32 sub-block sums of its row against
// four entries.  S1 = sum_j sc_j * D_j follows on the vector ALU; S2 = sum_j m_j * s_j takes
// two more products (the l and h bytes of the entry sums against the row's mins,
// S2 = D_l + 128 D_h).  The lane then folds the super-block term of its row and four entries
// into its accumulators (gemv.rs:539-547).

struct WStage {  // one super-block of the lane's weight row, as loaded
    v4u hdr;     // d, dmin | 12 scale bytes
    v4u x0, x1;  // code chunks (group 2(p&1), half p>>1) and (group 2(p&1)+1, half p>>1)
};
struct TStage {  // one super-block of the lane's entries, from global memory
    v4u lh;         // sub-block sums of entry c: l bytes, h bytes
    v4f dx;         // Q8_K scales of entries 4p + i
};

// One super-block of the lane's row in three 16-byte loads: the header and two code chunks,
// so the wavefront's loads cover its rows' 128 code bytes once.  A half-group holds k parts
// 2h and 2h + 1; swapping the second part of even rows (p = 0, 2) with the first part of odd
// rows (p = 1, 3) leaves every lane with k part p of all four groups.
SYN_DEV void load_w(const uint8_t* __restrict__ base, uint32_t off, uint32_t coff, WStage& w) {
    w.hdr = *reinterpret_cast<const v4u*>(base + off);
    w.x0 = *reinterpret_cast<const v4u*>(base + (off + coff));
    w.x1 = *reinterpret_cast<const v4u*>(base + (off + coff + 32));
}
// q[2g], q[2g + 1]: k part p of group g (odd rows' low words <-> even rows' high words, by
// v_permlane16_swap)
SYN_DEV void part_codes(const WStage& w, uint32_t (&q)[8]) {
    const auto r0 = __builtin_amdgcn_permlane16_swap(w.x0.x, w.x0.z, false, false);
    const auto r1 = __builtin_amdgcn_permlane16_swap(w.x0.y, w.x0.w, false, false);
    const auto r2 = __builtin_amdgcn_permlane16_swap(w.x1.x, w.x1.z, false, false);
    const auto r3 = __builtin_amdgcn_permlane16_swap(w.x1.y, w.x1.w, false, false);
    q[0] = r0[0];
    q[1] = r1[0];
    q[2] = r2[0];
    q[3] = r3[0];
    q[4] = r0[1];
    q[5] = r1[1];
    q[6] = r2[1];
    q[7] = r3[1];
}

SYN_DEV void load_t(const MoeAct& a, uint32_t lh_off, const float* __restrict__ d_row, TStage& t) {
    t.lh = *reinterpret_cast<const v4u*>(a.lh + lh_off);
    __builtin_memcpy(&t.dx, d_row, sizeof(t.dx));  // 4-byte aligned: the target picks the load width
}

// The entries' codes of one super-block in LDS: [entry c][k part p][sub-block j][8], rows of
// 272 bytes (the 16-byte pad spreads the 16 entries over the banks).
constexpr int TOK_STRIDE = 272;
constexpr int TOK_BUF = 16 * TOK_STRIDE;

SYN_DEV v4u tok_fetch(const MoeAct& a, int k, int b, int ent0, int nent) {
    const int t = threadIdx.x, c = t >> 4, u = t & 15;
    const int ec = ent0 + (c < nent ? c : nent - 1);
    return *reinterpret_cast<const v4u*>(a.codes + ((uint32_t)ec * (uint32_t)k + 256u * (uint32_t)b + 16u * (uint32_t)u));
}
SYN_DEV void tok_put(uint8_t* buf, v4u v) {
    const int t = threadIdx.x;
    *reinterpret_cast<v4u*>(buf + (t >> 4) * TOK_STRIDE + 16 * (t & 15)) = v;
}

SYN_DEV long pack2(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

SYN_DEV long q4k_codes(const uint32_t (&q)[8], int j) {
    const uint32_t lo = q[2 * (j >> 1)], hi = q[2 * (j >> 1) + 1];
    const uint32_t c0 = (j & 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
    const uint32_t c1 = (j & 1) ? (hi >> 4) & 0x0F0F0F0Fu : hi & 0x0F0F0F0Fu;
    return pack2(c0, c1);
}

// One super-block of NM weight rows (gate and up: NM = 2) against the item's entries.  The
// scheduling barriers and the pinned partial sums keep at most two sub-blocks' products
// live: sub-block j's products issue while sub-block j - 1's are scaled.
template <int NM>
SYN_DEV void q4k_super(const WStage (&w)[NM], const TStage& t, const uint8_t* tok, int p,
                       float (&acc)[NM][4]) {
    const int c = threadIdx.x & 15;
    v4u am[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) am[q] = *reinterpret_cast<const v4u*>(tok + c * TOK_STRIDE + 64 * p + 16 * q);
    uint32_t qs[NM][8], scs[NM][2], mns[NM][2];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        part_codes(w[m], qs[m]);
        // get_scale_min_k4 (gemv.rs:528-537) on packed bytes: scales of sub-blocks 0-3 | 4-7,
        // mins of sub-blocks 0-3 | 4-7
        const uint32_t w0 = w[m].hdr.y, w1 = w[m].hdr.z, w2 = w[m].hdr.w;
        scs[m][0] = w0 & 0x3F3F3F3Fu;
        scs[m][1] = (w2 & 0x0F0F0F0Fu) | ((w0 >> 2) & 0x30303030u);
        mns[m][0] = w1 & 0x3F3F3F3Fu;
        mns[m][1] = ((w2 >> 4) & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    }
    const v4i z = {0, 0, 0, 0};
    int s1[NM][4];
    v4i prev[NM];
#pragma unroll
    for (int j = 0; j <= 8; ++j) {
        v4i cur[NM];
        if (j < 8) {
            const v4u aw = am[j >> 1];
            const long av = (j & 1) ? pack2(aw.z, aw.w) : pack2(aw.x, aw.y);
#pragma unroll
            for (int m = 0; m < NM; ++m)
                cur[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, q4k_codes(qs[m], j), z, 0, 0, 0);
        }
        if (j > 0) {
            const int jj = j - 1;
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const int sc = (int)((scs[m][jj >> 2] >> (8 * (jj & 3))) & 0xFFu);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // |D| <= 32 * 15 * 127 fits 24 bits: one v_mad_i32_i24
                    const int dv = (prev[m][i] << 8) >> 8;
                    s1[m][i] = (jj ? s1[m][i] : 0) + sc * dv;
                    asm volatile("" : "+v"(s1[m][i]));  // here, not re-associated to the end
                }
            }
        }
        if (j < 8) {
#pragma unroll
            for (int m = 0; m < NM; ++m) prev[m] = cur[m];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // S2: lanes of k part 0 carry the l (then h) bytes of their entry and the row's mins
    const long al = p == 0 ? pack2(t.lh.x, t.lh.y) : 0;
    const long ah = p == 0 ? pack2(t.lh.z, t.lh.w) : 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const long bm = p == 0 ? pack2(mns[m][0], mns[m][1]) : 0;
        const v4i dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, bm, z, 0, 0, 0);
        const v4i dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, bm, z, 0, 0, 0);
        const float d = f16_to_f32(w[m].hdr.x), dmin = f16_to_f32(w[m].hdr.x >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int s2 = dl[i] + 128 * dh[i];
            const float dx = t.dx[i];
            acc[m][i] = acc[m][i] + ((d * dx) * (float)s1[m][i] - (dmin * dx) * (float)s2);
        }
    }
}

// The super-blocks of NM weight rows against the item's entries, in order.  Weights and the
// entries' sums and scales ping-pong between two register stages; the entries' codes between
// two LDS buffers, each filled by the whole workgroup one super-block ahead.  bases: the
// expert's matrices (wave-uniform); w_off: the lane's row.
template <int NM>
SYN_DEV void ffn_rows(const uint8_t* const (&bases)[NM], uint32_t w_off, const MoeAct& a, int k,
                      int ent0, int nent, int p, uint8_t* tok, float (&acc)[NM][4]) {
    const int nb = k / 256;
    const int c = threadIdx.x & 15;
    const int ent_a = ent0 + (c < nent ? c : nent - 1);
    const uint32_t coff = 16u + 64u * (uint32_t)(p & 1) + 16u * (uint32_t)(p >> 1);
    const uint32_t l0 = (uint32_t)ent_a * (uint32_t)nb * 16u;
    const float* d0 = a.d + ent0 + 4 * p;  // four output entries; the array is padded past its end
    const int64_t dstride = a.nentries;
    uint8_t* const tb0 = tok;
    uint8_t* const tb1 = tok + TOK_BUF;
    WStage wa[NM], wb[NM];
    TStage ta, tb;
    tok_put(tb0, tok_fetch(a, k, 0, ent0, nent));
#pragma unroll
    for (int m = 0; m < NM; ++m) load_w(bases[m], w_off, coff, wa[m]);
    load_t(a, l0, d0, ta);
    __syncthreads();
    // Pairs of super-blocks, every load and product unconditional inside the loop (a load
    // whose only use sat under a branch would sink to that use and stop flying early); the
    // odd last block, already in stage a, after it.
#pragma unroll 1
    for (int b = 0; b + 1 < nb; b += 2) {
        const uint32_t b1 = (uint32_t)(b + 1);
        const v4u n1 = tok_fetch(a, k, b1, ent0, nent);
#pragma unroll
        for (int m = 0; m < NM; ++m) load_w(bases[m], w_off + 144u * b1, coff, wb[m]);
        load_t(a, l0 + 16u * b1, d0 + dstride * b1, tb);
        __builtin_amdgcn_sched_barrier(0);
        q4k_super<NM>(wa, ta, tb0, p, acc);
        tok_put(tb1, n1);
        __syncthreads();
        // the next pair's first block; past the end, the last block again
        const uint32_t b2 = (uint32_t)(b + 2 < nb ? b + 2 : nb - 1);
        const v4u n2 = tok_fetch(a, k, b2, ent0, nent);
#pragma unroll
        for (int m = 0; m < NM; ++m) load_w(bases[m], w_off + 144u * b2, coff, wa[m]);
        load_t(a, l0 + 16u * b2, d0 + dstride * b2, ta);
        __builtin_amdgcn_sched_barrier(0);
        q4k_super<NM>(wb, tb, tb1, p, acc);
        tok_put(tb0, n2);
        __syncthreads();
    }
    if (nb & 1) {
        q4k_super<NM>(wa, ta, tb0, p, acc);
    }
}

// Entry range of expert e's items: offsets[e]..offsets[e+1].
struct MoeItems {
    const uint32_t* offsets;
    int n_experts;
    int row_groups;  // weight rows / 64
};
constexpr int MOE_CHUNK = 16;  // entries per item

// Maps a flat item index to (expert, row group, entry chunk); items of an expert with fewer
// entries are empty.  Items: expert-major, then entry chunk, then row group.  The item space,
// n_experts * row_groups * max_chunks, is sized on the device from the largest expert.
SYN_DEV int moe_max_chunks(const uint32_t* err) {
    const int most = (int)err[1];
    return (most + MOE_CHUNK - 1) / MOE_CHUNK;
}
SYN_DEV bool moe_item(const MoeItems& it, int item, int max_chunks, int& e, int& rg, int& ent0,
                      int& nent) {
    const int per_e = it.row_groups * max_chunks;
    e = item / per_e;
    const int r = item - e * per_e;
    const int ch = r / it.row_groups;
    rg = r - ch * it.row_groups;
    if (e >= it.n_experts) return false;
    const int b0 = (int)it.offsets[e], b1 = (int)it.offsets[e + 1];
    ent0 = b0 + ch * MOE_CHUNK;
    if (ent0 >= b1) return false;
    nent = b1 - ent0 < MOE_CHUNK ? b1 - ent0 : MOE_CHUNK;
    return true;
}

// gate/up + SiLU: h[entry][row] = silu(gate_row . x) * (up_row . x) (moe.rs:466-499).
__global__ __launch_bounds__(256, 3) void k_moe_gateup(const uint8_t* __restrict__ gate,
                                                       const uint8_t* __restrict__ up, int inter,
                                                       int hidden, MoeItems it, MoeAct a,
                                                       const uint32_t* __restrict__ err,
                                                       float* __restrict__ h) {
    __shared__ __attribute__((aligned(16))) uint8_t tok[2 * TOK_BUF];
    if (err[0]) return;
    const int max_chunks = moe_max_chunks(err);
    const int total = it.n_experts * it.row_groups * max_chunks;
    const int lane = threadIdx.x & 63, p = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row_bytes = (uint32_t)(hidden / 256) * 144u;
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        int e, rg, ent0, nent;
        if (!moe_item(it, item, max_chunks, e, rg, ent0, nent)) continue;  // uniform per workgroup
        const int row = rg * 64 + wave * 16 + (lane & 15);
        const int64_t ebytes = (int64_t)inter * row_bytes;
        const uint8_t* const bases[2] = {gate + e * ebytes, up + e * ebytes};
        float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        ffn_rows<2>(bases, (uint32_t)row * row_bytes, a, hidden, ent0, nent, p, tok, acc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * p + i < nent)
                h[(int64_t)(ent0 + 4 * p + i) * inter + row] = ref_silu(acc[0][i]) * acc[1][i];
        __syncthreads();  // the LDS buffers are refilled by the next item
    }
}

// down: out[slot][row] = down_row . hq[entry], written to the entry's slot (the reference's
// scatter, moe.rs:501-515).
__global__ __launch_bounds__(256, 3) void k_moe_down(const uint8_t* __restrict__ down, int hidden,
                                                     int inter, MoeItems it, MoeAct a,
                                                     const uint32_t* __restrict__ slots,
                                                     const uint32_t* __restrict__ err,
                                                     float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint8_t tok[2 * TOK_BUF];
    if (err[0]) return;
    const int max_chunks = moe_max_chunks(err);
    const int total = it.n_experts * it.row_groups * max_chunks;
    const int lane = threadIdx.x & 63, p = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row_bytes = (uint32_t)(inter / 256) * 144u;
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        int e, rg, ent0, nent;
        if (!moe_item(it, item, max_chunks, e, rg, ent0, nent)) continue;  // uniform per workgroup
        const int row = rg * 64 + wave * 16 + (lane & 15);
        const uint8_t* const bases[1] = {down + e * ((int64_t)hidden * row_bytes)};
        float acc[1][4] = {{0.0f, 0.0f, 0.0f, 0.0f}};
        ffn_rows<1>(bases, (uint32_t)row * row_bytes, a, inter, ent0, nent, p, tok, acc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * p + i < nent) out[(int64_t)slots[ent0 + 4 * p + i] * hidden + row] = acc[0][i];
        __syncthreads();  // the LDS buffers are refilled by the next item
    }
}

// The grid covers every item of the common case (the largest expert within one entry chunk)
// with one workgroup each; larger item spaces, sized on the device, are walked grid-stride.
static unsigned moe_grid(int n_experts, int row_groups, int nentries) {
    int64_t items = (int64_t)n_experts * row_groups;
    const int64_t cap = (int64_t)n_experts * row_groups * ((nentries + MOE_CHUNK - 1) / MOE_CHUNK);
    items = items < cap ? items : cap;
    return (unsigned)(items > 0 ? items : 1);
}

void launch_moe_gateup(const uint8_t* gate, const uint8_t* up, int n_experts, int hidden,
                       int inter, const uint32_t* offsets, int nentries, MoeAct a,
                       const uint32_t* err, float* h, hipStream_t stream) {
    MoeItems it{offsets, n_experts, inter / 64};
    hipLaunchKernelGGL(k_moe_gateup, dim3(moe_grid(n_experts, it.row_groups, nentries)), dim3(256), 0,
                       stream, gate, up, inter, hidden, it, a, err, h);
}

void launch_moe_down(const uint8_t* down, int n_experts, int hidden, int inter,
                     const uint32_t* offsets, int nentries, MoeAct a, const uint32_t* slots,
                     const uint32_t* err, float* out, hipStream_t stream) {
    MoeItems it{offsets, n_experts, hidden / 64};
    hipLaunchKernelGGL(k_moe_down, dim3(moe_grid(n_experts, it.row_groups, nentries)), dim3(256), 0,
                       stream, down, hidden, inter, it, a, slots, err, out);
}

// ============================================================================================
// MoeCombine (moe/tests.rs:541-556)
// ============================================================================================

// One workgroup per (row, 1024 columns); the row's slots are ordered by expert id (stable)
// once in LDS, then each thread adds its columns in that order.
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ out,
                                                     const int32_t* __restrict__ ids,
                                                     const float* __restrict__ w, int top_k,
                                                     int hidden, float* __restrict__ y) {
    __shared__ int order[64];
    const int r = blockIdx.y;
    if (threadIdx.x == 0) {
        for (int j = 0; j < top_k; ++j) order[j] = j;
        for (int a2 = 1; a2 < top_k; ++a2) {  // stable insertion sort by id
            const int v = order[a2];
            int b2 = a2;
            while (b2 > 0 && ids[(int64_t)r * top_k + order[b2 - 1]] > ids[(int64_t)r * top_k + v]) {
                order[b2] = order[b2 - 1];
                --b2;
            }
            order[b2] = v;
        }
    }
    __syncthreads();
    for (int c = blockIdx.x * 1024 + threadIdx.x; c < hidden && c < (int)(blockIdx.x + 1) * 1024; c += 256) {
        float acc = 0.0f;
        for (int a2 = 0; a2 < top_k; ++a2) {
            const int j = order[a2];
            const float wj = w[(int64_t)r * top_k + j];
            acc = acc + wj * out[((int64_t)r * top_k + j) * hidden + c];
        }
        y[(int64_t)r * hidden + c] = acc;
    }
}

void launch_moe_combine(const float* out, const int32_t* ids, const float* w, int rows, int top_k,
                        int hidden, float* y, hipStream_t stream) {
    if (rows == 0 || hidden == 0) return;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((hidden + 1023) / 1024), (unsigned)rows),
                       dim3(256), 0, stream, out, ids, w, top_k, hidden, y);
}

}  // namespace syn
