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

// ============================================================================================
// MoeRoute{Softmax}
// ============================================================================================

// One workgroup per TT tokens.  Logits: the block sums of EC experts at a time go to LDS, then
// the pairwise tree runs level by level in LDS (ping-pong), exactly as reduce.rs defines.
template <int TT>
__global__ __launch_bounds__(256) void k_moe_route(const float* __restrict__ router,
                                                   const float* __restrict__ x, int rows,
                                                   int hidden, int n_experts, int top_k,
                                                   int renorm, int32_t* __restrict__ ids,
                                                   float* __restrict__ wout,
                                                   float* __restrict__ probs_out) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * TT;
    const int nblk = hidden / 32;
    constexpr int EC = 8;  // experts per chunk
    float* xs = sm;                                   // [TT][hidden]
    float* logit = xs + TT * hidden;                  // [TT][n_experts]
    float* S0 = logit + TT * n_experts;               // [TT][EC][nblk]
    float* S1 = S0 + TT * EC * nblk;                  // [TT][EC][nblk]
    for (int i = tid; i < TT * hidden; i += 256) {
        const int t = i / hidden, c = i - t * hidden;
        xs[i] = (t0 + t < rows) ? x[(int64_t)(t0 + t) * hidden + c] : 0.0f;
    }
    __syncthreads();
    for (int e0 = 0; e0 < n_experts; e0 += EC) {
        const int ec = n_experts - e0 < EC ? n_experts - e0 : EC;
        // block sums: thread per (expert, block), all TT tokens
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
                const float* s = src + (t * EC + e) * nblk;
                dst[(t * EC + e) * nblk + i] = (2 * i + 1 < n) ? s[2 * i] + s[2 * i + 1] : s[2 * i];
            }
            __syncthreads();
            float* tmp = src;
            src = dst;
            dst = tmp;
        }
        for (int p = tid; p < TT * ec; p += 256) {
            const int t = p / ec, e = p - t * ec;
            logit[t * n_experts + e0 + e] = nblk > 0 ? src[(t * EC + e) * nblk] : 0.0f;
        }
        __syncthreads();
    }
    // softmax and top-k: one wavefront per token
    const int lane = tid & 63, wave = tid >> 6;
    for (int t = wave; t < TT; t += 4) {
        if (t0 + t >= rows) continue;
        float* lg = logit + t * n_experts;
        float m = -__builtin_inff();
        bool first = true;
        for (int e = lane; e < n_experts; e += 64) {
            if (first || lg[e] > m) m = lg[e];
            first = false;
        }
        // row maximum (order-free); lanes with no expert hold -inf
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float o = __shfl_xor(m, off);
            m = o > m ? o : m;
        }
        for (int e = lane; e < n_experts; e += 64) lg[e] = ref_exp(lg[e] - m);
        wave_lds_sync();
        // F32Fixed sum of the E exponentials: one lane streams the reduce.rs tree
        float total = 0.0f;
        if (lane == 0) {
            float sums[16];
            int lv[16];
            int depth = 0;
            for (int s0 = 0; s0 < n_experts; s0 += 32) {
                float acc = 0.0f;
                const int s1 = n_experts < s0 + 32 ? n_experts : s0 + 32;
                for (int i = s0; i < s1; ++i) acc = acc + lg[i];
                int level = 0;
                while (depth > 0 && lv[depth - 1] == level) {
                    depth -= 1;
                    acc = sums[depth] + acc;
                    level += 1;
                }
                sums[depth] = acc;
                lv[depth] = level;
                depth += 1;
            }
            if (depth > 0) {
                total = sums[depth - 1];
                for (int i = depth - 2; i >= 0; --i) total = sums[i] + total;
            }
        }
        total = __shfl(total, 0);
        for (int e = lane; e < n_experts; e += 64) lg[e] = lg[e] / total;
        wave_lds_sync();
        if (probs_out)
            for (int e = lane; e < n_experts; e += 64) probs_out[(int64_t)(t0 + t) * n_experts + e] = lg[e];
        // top-k: k rounds of (probability desc, index asc); taken experts are skipped
        uint64_t taken[4] = {0, 0, 0, 0};  // n_experts <= 256
        float sel[32];
        int sid[32];
        for (int j = 0; j < top_k; ++j) {
            float bv = 0.0f;
            int bi = 0x7FFFFFFF;
            for (int e = lane; e < n_experts; e += 64) {
                if ((taken[e >> 6] >> (e & 63)) & 1) continue;
                const float v = lg[e];
                if (bi == 0x7FFFFFFF || v > bv) {
                    bv = v;
                    bi = e;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float ov = __shfl_xor(bv, off);
                const int oi = __shfl_xor(bi, off);
                const bool better = (oi != 0x7FFFFFFF) &&
                                    (bi == 0x7FFFFFFF || ov > bv || (ov == bv && oi < bi));
                if (better) {
                    bv = ov;
                    bi = oi;
                }
            }
            taken[bi >> 6] |= 1ull << (bi & 63);
            sel[j] = bv;
            sid[j] = bi;
        }
        if (lane == 0) {
            float tsum = 0.0f;
            for (int j = 0; j < top_k; ++j) tsum = tsum + sel[j];  // one block: in order from +0
            for (int j = 0; j < top_k; ++j) {
                ids[(int64_t)(t0 + t) * top_k + j] = sid[j];
                wout[(int64_t)(t0 + t) * top_k + j] = renorm ? sel[j] / tsum : sel[j];
            }
        }
    }
}

size_t moe_route_lds(int tt, int hidden, int n_experts) {
    return sizeof(float) * ((size_t)tt * hidden + (size_t)tt * n_experts + 2ull * tt * 8 * (hidden / 32));
}

void launch_moe_route(const float* router, const float* x, int rows, int hidden, int n_experts,
                      int top_k, int renorm, int32_t* ids, float* w, float* probs,
                      hipStream_t stream) {
    // Several tokens per workgroup share each router block once there are enough tokens and
    // their rows fit the 64 KB of LDS a launch asks for.
    constexpr size_t LDS_MAX = 64 * 1024;
    if (rows >= 512 && moe_route_lds(4, hidden, n_experts) <= LDS_MAX) {
        hipLaunchKernelGGL((k_moe_route<4>), dim3((rows + 3) / 4), dim3(256),
                           moe_route_lds(4, hidden, n_experts), stream, router, x, rows, hidden,
                           n_experts, top_k, renorm, ids, w, probs);
    } else if (rows >= 512 && moe_route_lds(2, hidden, n_experts) <= LDS_MAX) {
        hipLaunchKernelGGL((k_moe_route<2>), dim3((rows + 1) / 2), dim3(256),
                           moe_route_lds(2, hidden, n_experts), stream, router, x, rows, hidden,
                           n_experts, top_k, renorm, ids, w, probs);
    } else {
        hipLaunchKernelGGL((k_moe_route<1>), dim3(rows), dim3(256),
                           moe_route_lds(1, hidden, n_experts), stream, router, x, rows, hidden,
                           n_experts, top_k, renorm, ids, w, probs);
    }
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
    // scan: expert-major, wave-minor
    if (tid == 0) {
        uint32_t run = 0, most = 0;
        for (int e = 0; e < n_experts; ++e) {
            offsets[e] = run;
            const uint32_t start = run;
            for (int w = 0; w < 16; ++w) {
                const uint32_t c = cnt[w * n_experts + e];
                cnt[w * n_experts + e] = run;
                run += c;
            }
            most = run - start > most ? run - start : most;
        }
        offsets[n_experts] = run;
        err[0] = 0u;
        err[1] = most;  // the largest expert's entry count, which sizes the FFN item space
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

// One wavefront per (entry, 256-value block).
__global__ __launch_bounds__(256) void k_moe_gather_q8k(const float* __restrict__ x,
                                                        const uint32_t* __restrict__ slots,
                                                        int nentries, int top_k, int k,
                                                        const uint32_t* __restrict__ err,
                                                        int8_t* __restrict__ codes,
                                                        float* __restrict__ d,
                                                        int32_t* __restrict__ sums, int gather) {
    if (err[0]) return;
    const int nb = k / 256;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (int64_t)nentries * nb) return;
    const int i = (int)(item / nb), b = (int)(item - (int64_t)i * nb);
    const int64_t src_row = gather ? (int64_t)(slots[i] / (uint32_t)top_k) : i;
    q8k_block_wave(x + src_row * k + (int64_t)b * 256, codes + (int64_t)i * k + (int64_t)b * 256,
                   d + (int64_t)i * nb + b, sums + (int64_t)i * (k / 32) + (int64_t)b * 8,
                   threadIdx.x & 63);
}

void launch_moe_gather_q8k(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                           const uint32_t* err, int8_t* codes, float* d, int32_t* sums, int gather,
                           hipStream_t stream) {
    const int64_t items = (int64_t)nentries * (k / 256);
    if (items == 0) return;
    hipLaunchKernelGGL(k_moe_gather_q8k, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, x,
                       slots, nentries, top_k, k, err, codes, d, sums, gather);
}

// ============================================================================================
// Grouped Q4_K product on the int8 matrix cores
// ============================================================================================
//
// A work item is (expert, 16 consecutive weight rows, up to TB*16 consecutive entries of the
// expert).  Lane l: weight row l%16 of the tile (B operand), token l%16 of a 16-token block
// (A operand), k part p = l/16; outputs D[token 4p+i][row l%16], i = 0..3.

// Exact per-sub-block I32 sums of one super-block for one 16-token block, then the F32 term
// folded into acc[i] (gemv.rs:539-547) for the lane's 4 tokens.
SYN_DEV void q4k_mfma_superblock(const uint32_t (&qw)[8], int sc_lo_hi_dummy, const int* sc,
                                 const int* mn, float d, float dmin, const QAct& a,
                                 int64_t kcodes, int nb, int b, int ent0, int nent, int lane,
                                 float* acc) {
    const int p = lane >> 4, tcol = lane & 15;
    // A operands: token ent0 + tcol, elements 32j + 8p .. +7 of super-block b
    const int ent_a = ent0 + tcol;
    const bool a_ok = tcol < nent;
    const int8_t* xa = a.codes + (int64_t)(a_ok ? ent_a : ent0) * kcodes + (int64_t)b * 256 + 8 * p;
    v4i r = {0, 0, 0, 0};
    int s1[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        long av = a_ok ? *reinterpret_cast<const long*>(xa + 32 * j) : 0;
        // weight codes of sub-block j: nibble (j & 1) of the lane's 8 bytes of group j/2
        const uint32_t lo = qw[2 * (j >> 1)], hi = qw[2 * (j >> 1) + 1];
        const uint32_t c0 = (j & 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
        const uint32_t c1 = (j & 1) ? (hi >> 4) & 0x0F0F0F0Fu : hi & 0x0F0F0F0Fu;
        const long bv = (long)(((uint64_t)c1 << 32) | c0);
        const v4i z = {0, 0, 0, 0};
        r = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, z, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) s1[i] += sc[j] * r[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ent = ent0 + 4 * p + i;
        if (4 * p + i < nent) {
            const int4* xs = reinterpret_cast<const int4*>(a.sums + (int64_t)ent * (kcodes / 32) + (int64_t)b * 8);
            const int4 u = xs[0], v = xs[1];
            const int s2 = mn[0] * u.x + mn[1] * u.y + mn[2] * u.z + mn[3] * u.w + mn[4] * v.x +
                           mn[5] * v.y + mn[6] * v.z + mn[7] * v.w;
            const float dx = a.d[(int64_t)ent * nb + b];
            acc[i] = acc[i] + ((d * dx) * (float)s1[i] - (dmin * dx) * (float)s2);
        }
    }
}

// Weight data of one super-block for the lane's row: header words and the lane's 8 bytes of
// each of the four 32-byte code groups.
SYN_DEV void load_q4k_lane(const uint8_t* __restrict__ rowp, int b, int p, v4u& hdr, uint32_t (&qw)[8]) {
    const uint8_t* blk = rowp + (int64_t)b * 144;
    hdr = *reinterpret_cast<const v4u*>(blk);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint2 v = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + 8 * p);
        qw[2 * g] = v.x;
        qw[2 * g + 1] = v.y;
    }
}

// Entry range of expert e's items: offsets[e]..offsets[e+1].
struct MoeItems {
    const uint32_t* offsets;
    int n_experts;
    int row_tiles;   // weight rows / 16
    int ent_chunk;   // entries per item (multiple of 16)
};

// Maps a flat item index to (expert, row tile, entry chunk); items of an expert with fewer
// entries are empty.  Items: expert-major, then entry chunk, then row tile.  The item space,
// n_experts * row_tiles * max_chunks, is sized on the device from the largest expert.
SYN_DEV int moe_max_chunks(const MoeItems& it, const uint32_t* err) {
    const int most = (int)err[1];
    return most > 0 ? (most + it.ent_chunk - 1) / it.ent_chunk : 0;
}
SYN_DEV bool moe_item(const MoeItems& it, int item, int max_chunks, int& e, int& rt, int& ent0,
                      int& nent) {
    const int per_e = it.row_tiles * max_chunks;
    e = item / per_e;
    const int r = item - e * per_e;
    const int ch = r / it.row_tiles;
    rt = r - ch * it.row_tiles;
    if (e >= it.n_experts) return false;
    const int b0 = (int)it.offsets[e], b1 = (int)it.offsets[e + 1];
    ent0 = b0 + ch * it.ent_chunk;
    if (ent0 >= b1) return false;
    nent = b1 - ent0 < it.ent_chunk ? b1 - ent0 : it.ent_chunk;
    return true;
}

// gate/up + SiLU: h[entry][row] = silu(gate_row . x) * (up_row . x) for the item's rows and
// entries.  TB = 16-token blocks per item.
template <int TB>
SYN_DEV void gateup_item(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                         int inter, int hidden, const MoeItems& it, int max_chunks, const QAct& a,
                         int item, float* __restrict__ h) {
    const int lane = threadIdx.x & 63;
    int e, rt, ent0, nent;
    if (!moe_item(it, item, max_chunks, e, rt, ent0, nent)) return;
    const int nb = hidden / 256, p = lane >> 4;
    const int row = rt * 16 + (lane & 15);
    const int64_t row_bytes = (int64_t)nb * 144;
    const int64_t ebytes = (int64_t)inter * row_bytes;
    const uint8_t* grow = gate + (int64_t)e * ebytes + (int64_t)row * row_bytes;
    const uint8_t* urow = up + (int64_t)e * ebytes + (int64_t)row * row_bytes;
    float ag[TB][4], au[TB][4];
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) ag[t][i] = au[t][i] = 0.0f;
    for (int b = 0; b < nb; ++b) {
        v4u hg, hu;
        uint32_t qg[8], qu[8];
        load_q4k_lane(grow, b, p, hg, qg);
        load_q4k_lane(urow, b, p, hu, qu);
        int scg[8], mng[8], scu[8], mnu[8];
        scales_k4(hg.y, hg.z, hg.w, scg, mng);
        scales_k4(hu.y, hu.z, hu.w, scu, mnu);
        const float dg = f16_to_f32(hg.x), dming = f16_to_f32(hg.x >> 16);
        const float du = f16_to_f32(hu.x), dminu = f16_to_f32(hu.x >> 16);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int e0 = ent0 + 16 * t;
            const int ne = nent - 16 * t;
            if (ne <= 0) break;
            q4k_mfma_superblock(qg, 0, scg, mng, dg, dming, a, hidden, nb, b, e0, ne, lane, ag[t]);
            q4k_mfma_superblock(qu, 0, scu, mnu, du, dminu, a, hidden, nb, b, e0, ne, lane, au[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = 16 * t + 4 * p + i;
            if (idx < nent) h[(int64_t)(ent0 + idx) * inter + row] = ref_silu(ag[t][i]) * au[t][i];
        }
}


template <int TB>
__global__ __launch_bounds__(256) void k_moe_gateup(const uint8_t* __restrict__ gate,
                                                    const uint8_t* __restrict__ up, int inter,
                                                    int hidden, MoeItems it, QAct a,
                                                    const uint32_t* __restrict__ err,
                                                    float* __restrict__ h) {
    if (err[0]) return;
    const int max_chunks = moe_max_chunks(it, err);
    const int total = it.n_experts * it.row_tiles * max_chunks;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4)
        gateup_item<TB>(gate, up, inter, hidden, it, max_chunks, a, item, h);
}
// down: out[slot][row] = down_row . hq[entry] for the item's rows and entries, written to
// the entry's slot (the reference's scatter, moe.rs:501-515).
template <int TB>
SYN_DEV void down_item(const uint8_t* __restrict__ down, int hidden, int inter,
                       const MoeItems& it, int max_chunks, const QAct& a,
                       const uint32_t* __restrict__ slots, int item, float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    int e, rt, ent0, nent;
    if (!moe_item(it, item, max_chunks, e, rt, ent0, nent)) return;
    const int nb = inter / 256, p = lane >> 4;
    const int row = rt * 16 + (lane & 15);
    const int64_t row_bytes = (int64_t)nb * 144;
    const uint8_t* drow = down + (int64_t)e * hidden * row_bytes + (int64_t)row * row_bytes;
    float ad[TB][4];
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) ad[t][i] = 0.0f;
    for (int b = 0; b < nb; ++b) {
        v4u hd;
        uint32_t qd[8];
        load_q4k_lane(drow, b, p, hd, qd);
        int sc[8], mn[8];
        scales_k4(hd.y, hd.z, hd.w, sc, mn);
        const float dd = f16_to_f32(hd.x), dmin = f16_to_f32(hd.x >> 16);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int e0 = ent0 + 16 * t;
            const int ne = nent - 16 * t;
            if (ne <= 0) break;
            q4k_mfma_superblock(qd, 0, sc, mn, dd, dmin, a, inter, nb, b, e0, ne, lane, ad[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = 16 * t + 4 * p + i;
            if (idx < nent) out[(int64_t)slots[ent0 + idx] * hidden + row] = ad[t][i];
        }
}

template <int TB>
__global__ __launch_bounds__(256) void k_moe_down(const uint8_t* __restrict__ down, int hidden,
                                                  int inter, MoeItems it, QAct a,
                                                  const uint32_t* __restrict__ slots,
                                                  const uint32_t* __restrict__ err,
                                                  float* __restrict__ out) {
    if (err[0]) return;
    const int max_chunks = moe_max_chunks(it, err);
    const int total = it.n_experts * it.row_tiles * max_chunks;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4)
        down_item<TB>(down, hidden, inter, it, max_chunks, a, slots, item, out);
}

// Items per expert: ceil(max entries of one expert / chunk) chunks x row tiles; the item count
// is sized for the worst case (every slot on one expert), empty items exit at once.
// The grid covers every item of the common case (the largest expert within one entry chunk)
// in one wavefront each; larger item spaces, sized on the device, are walked grid-stride.
static unsigned moe_grid(int n_experts, int row_tiles, int nentries, int chunk) {
    int64_t items = (int64_t)n_experts * row_tiles;
    const int64_t cap = (int64_t)n_experts * row_tiles * ((nentries + chunk - 1) / chunk);
    items = items < cap ? items : cap;
    if (items < 4) items = 4;
    return (unsigned)((items + 3) / 4);
}

void launch_moe_gateup(const uint8_t* gate, const uint8_t* up, int n_experts, int hidden,
                       int inter, const uint32_t* offsets, int nentries, QAct a,
                       const uint32_t* err, float* h, hipStream_t stream) {
    constexpr int TB = 4;
    MoeItems it{offsets, n_experts, inter / 16, 16 * TB};
    hipLaunchKernelGGL((k_moe_gateup<TB>), dim3(moe_grid(n_experts, it.row_tiles, nentries, it.ent_chunk)),
                       dim3(256), 0, stream, gate, up, inter, hidden, it, a, err, h);
}

void launch_moe_down(const uint8_t* down, int n_experts, int hidden, int inter,
                     const uint32_t* offsets, int nentries, QAct a, const uint32_t* slots,
                     const uint32_t* err, float* out, hipStream_t stream) {
    constexpr int TB = 4;
    MoeItems it{offsets, n_experts, hidden / 16, 16 * TB};
    hipLaunchKernelGGL((k_moe_down<TB>), dim3(moe_grid(n_experts, it.row_tiles, nentries, it.ent_chunk)),
                       dim3(256), 0, stream, down, hidden, inter, it, a, slots, err, out);
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
