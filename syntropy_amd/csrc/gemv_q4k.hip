// Decode GEMV for Q4_K weights, one activation row: the path's headline kernel.
//
// Value: crates/kernels-cpu/src/gemv.rs:539-547 (q4k_term) folded in ascending super-block
// order from +0.0 (gemv/portable.rs:114-190), bit for bit.
//
// Design (gfx950):
//  * A wavefront owns one 4-row group: 16 lanes per output row, lane j takes super-blocks
//    j, j+16, j+32, ... ("rounds") of its row.  Each lane loads its 144-byte super-block straight
//    into registers with nine 16-byte loads; with more than one round the next round's block is
//    loaded into the other half of a register ping-pong before the current one is computed.
//    The rounds are unrolled and every load is unconditional (an idle lane reloads the matrix's
//    first block), so the compiler's wait counts stay exact and a wavefront always has a block
//    in flight.
//  * The weight loads of the first round are issued before the workgroup prepares the
//    activation row, so HBM latency overlaps that prologue.
//  * The activation row lives in LDS for the whole workgroup: quantized to Q8_K in the
//    prologue (FUSE = 1: the Gemv op, F32 row in, one launch) or copied from a workspace
//    quantized earlier (FUSE = 0).  Column c's codes sit at c*272 bytes (a 16-byte skew per
//    column), so the 16 columns a wavefront reads at once fall in distinct banks.
//  * The 16 terms of a row are folded in order by passing the running sum from lane to lane
//    with DPP row_ror:1, once per round.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

namespace {

constexpr int COL = 272;  // LDS bytes per activation column (256 codes + 16-byte skew)
constexpr int SUMW = 32;  // LDS bytes per column of 32-value sums (8 ints)

SYN_HD inline size_t q4k_dec_lds(int nb) { return (size_t)nb * (COL + SUMW + 4); }
SYN_DEV int xs_off(int nb) { return nb * COL; }
SYN_DEV int xd_off(int nb) { return nb * (COL + SUMW); }

template <int NT>
SYN_DEV v4u ldw(const uint8_t* p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    else
        return *reinterpret_cast<const v4u*>(p);
}

// Lane `part` = c % 16 of super-block c / 16's group of 16 lanes: values 16 part .. +15.
SYN_DEV void load_block16(const float* __restrict__ x, int c, float (&v)[16]) {
    const int sb = c >> 4, part = c & 15;
    const float4* src = reinterpret_cast<const float4*>(x + (int64_t)sb * 256 + part * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 a = src[q];
        v[4 * q] = a.x;
        v[4 * q + 1] = a.y;
        v[4 * q + 2] = a.z;
        v[4 * q + 3] = a.w;
    }
}

SYN_DEV void quant16_to_lds(const float (&v)[16], int c, int nb, uint8_t* lds) {
    const int sb = c >> 4, part = c & 15;
    // largest magnitude, the first index on a tie; any non-finite value in the 16 lanes
    float amax, mx;
    bool bad;
    block_signed_amax<16>(v, part * 16, amax, mx, bad);
    // codes of is v: is 0 where the codes are all 0 (an all-zero block, an infinite inverse
    // scale), which leaves finite values' codes 0; a block with a NaN or an infinity (`bad`) is
    // zeroed whole after the arithmetic (straight-line code: no branch around the 16 values)
    float d = 0.0f, is = 0.0f;
    if (bad) {
        d = __builtin_nanf("");
    } else if (amax != 0.0f) {
        const float iscale = neg127_div(mx);
        is = finite_f(iscale) ? iscale : 0.0f;  // |iscale v| <= 127 (to a rounding): nearest_int_small's range
        d = recip_rn(iscale);
    }
    int q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int n = nearest_int_small(is * v[i]);
        q[i] = n < 127 ? n : 127;
    }
    uint32_t w[4];
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = (uint32_t)(q[4 * k] & 0xFF) | ((uint32_t)(q[4 * k + 1] & 0xFF) << 8) |
               ((uint32_t)(q[4 * k + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * k + 3] & 0xFF) << 24);
        w[k] = bad ? 0u : w[k];
        s = sdot4(w[k], 0x01010101u, s);  // the four codes' sum, exact
    }
    v4u pk = {w[0], w[1], w[2], w[3]};
    *reinterpret_cast<v4u*>(lds + sb * COL + part * 16) = pk;
    s += (int)dpp_u32<DPP_XOR1>((uint32_t)s);  // the two 16-value halves of a 32-value group
    if ((part & 1) == 0) reinterpret_cast<int*>(lds + xs_off(nb) + sb * SUMW)[part >> 1] = s;
    if (part == 0) reinterpret_cast<float*>(lds + xd_off(nb))[sb] = d;
}

SYN_DEV void quant_block16(const float* __restrict__ x, int c, int nb, uint8_t* lds) {
    float v[16];
    load_block16(x, c, v);
    quant16_to_lds(v, c, nb, lds);
}

// Q8_K of the activation row into LDS (crates/kernels-cpu/src/gemv/act.rs:351-373): 16 lanes
// per 256-value super-block, 16 values per lane.  Largest magnitude, first index on ties.
SYN_DEV void quant_row_to_lds(const float* __restrict__ x, int nb, uint8_t* lds) {
    for (int c = threadIdx.x; c < nb * 16; c += blockDim.x)  // the 16 lanes of a super-block stay together
        quant_block16(x, c, nb, lds);
}

SYN_DEV void copy_row_to_lds(const int8_t* __restrict__ xq, const float* __restrict__ xd,
                             const int32_t* __restrict__ xs, int nb, uint8_t* lds) {
    for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
        const int c = i >> 4, p = i & 15;
        *reinterpret_cast<v4u*>(lds + c * COL + p * 16) =
            *reinterpret_cast<const v4u*>(xq + (int64_t)c * 256 + p * 16);
    }
    for (int i = threadIdx.x; i < nb * 2; i += blockDim.x) {
        const int c = i >> 1, p = i & 1;
        *reinterpret_cast<v4u*>(lds + xs_off(nb) + c * SUMW + p * 16) =
            *reinterpret_cast<const v4u*>(xs + (int64_t)c * 8 + p * 4);
    }
    for (int i = threadIdx.x; i < nb; i += blockDim.x) reinterpret_cast<float*>(lds + xd_off(nb))[i] = xd[i];
}

// One super-block's term from its nine 16-byte words and activation column b in LDS.
SYN_DEV float q4k_term_lds(const v4u* wv, const uint8_t* lds, int nb, int b) {
    uint32_t wb[36];
#pragma unroll
    for (int i = 0; i < 9; ++i) {
        wb[4 * i] = wv[i].x;
        wb[4 * i + 1] = wv[i].y;
        wb[4 * i + 2] = wv[i].z;
        wb[4 * i + 3] = wv[i].w;
    }
    int sc[8], mn[8];
    scales_k4(wb[1], wb[2], wb[3], sc, mn);
    const float d = f16_to_f32(wb[0]), dmin = f16_to_f32(wb[0] >> 16);
    const uint8_t* xc = lds + b * COL;
    int s1 = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const v4u xl0 = *reinterpret_cast<const v4u*>(xc + 64 * g);
        const v4u xl1 = *reinterpret_cast<const v4u*>(xc + 64 * g + 16);
        const v4u xh0 = *reinterpret_cast<const v4u*>(xc + 64 * g + 32);
        const v4u xh1 = *reinterpret_cast<const v4u*>(xc + 64 * g + 48);
        const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t q = wb[4 + 8 * g + t];
            lo = sdot4(q & 0x0F0F0F0Fu, xl[t], lo);
            hi = sdot4((q >> 4) & 0x0F0F0F0Fu, xh[t], hi);
        }
        s1 = mad24(sc[2 * g + 1], hi, mad24(sc[2 * g], lo, s1));
    }
    const int4 sa = *reinterpret_cast<const int4*>(lds + xs_off(nb) + b * SUMW);
    const int4 sb = *reinterpret_cast<const int4*>(lds + xs_off(nb) + b * SUMW + 16);
    const float dx = reinterpret_cast<const float*>(lds + xd_off(nb))[b];
    const int s2 = q4k_s2(mn, sa, sb);
    return (d * dx) * (float)s1 - (dmin * dx) * (float)s2;
}

}  // namespace

// The 4-row group of one wavefront: rows row0 + lane/16.  NR = ceil(nb / 16) rounds, fixed at
// compile time so the body is straight-line code.  `A` holds round 0, already in flight.
template <int NT, int NR>
SYN_DEV void rowgroup_body(const uint8_t* __restrict__ W, int n_out, int nb, int row,
                           const uint8_t* lds, v4u* A, float* __restrict__ y) {
    const int j = threadIdx.x & 15;
    const int64_t row_bytes = (int64_t)nb * 144;
    const bool row_ok = row < n_out;
    auto blk = [&](int r) {
        const int b = r * 16 + j;
        const bool ok = row_ok && b < nb;
        return ok ? W + (int64_t)row * row_bytes + (int64_t)b * 144 : W;
    };
    v4u B[9];
    float acc = 0.0f;
    auto consume = [&](const v4u* buf, int r) {
        const int b = r * 16 + j;
        const bool ok = row_ok && b < nb;
        const float t = q4k_term_lds(buf, lds, nb, ok ? b : 0);
        const float tv = ok ? t : 0.0f;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            acc = rot1<16>(acc);
            acc = acc + ((j == s) ? tv : 0.0f);
        }
    };
#pragma unroll
    for (int r = 0; r < NR; r += 2) {
        if (r + 1 < NR) {
            const uint8_t* p = blk(r + 1);
#pragma unroll
            for (int i = 0; i < 9; ++i) B[i] = ldw<NT>(p + 16 * i);
        }
        consume(A, r);
        if (r + 2 < NR) {
            const uint8_t* p = blk(r + 2);
#pragma unroll
            for (int i = 0; i < 9; ++i) A[i] = ldw<NT>(p + 16 * i);
        }
        if (r + 1 < NR) consume(B, r + 1);
    }
    if (j == 15 && row_ok) y[row] = acc;
}

template <int NT>
SYN_DEV void load_round0(const uint8_t* __restrict__ W, int n_out, int nb, int row, v4u* A) {
    const int j = threadIdx.x & 15;
    const bool ok = row < n_out && j < nb;
    const uint8_t* p = ok ? W + (int64_t)row * nb * 144 + (int64_t)j * 144 : W;
#pragma unroll
    for (int i = 0; i < 9; ++i) A[i] = ldw<NT>(p + 16 * i);
}

template <int FUSE, int NT, int NR>
__global__ __launch_bounds__(256) void k_gemv_q4k_dec(const uint8_t* __restrict__ W, int n_out,
                                                      int nb, const float* __restrict__ xf,
                                                      const int8_t* __restrict__ xq,
                                                      const float* __restrict__ xd,
                                                      const int32_t* __restrict__ xs,
                                                      float* __restrict__ y,
                                                      const uint32_t* __restrict__ active) {
    if (active_rows(active, 0, 1) == 0) return;  // a step with no active row
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * 4 + wave) * 4 + (lane >> 4);
    v4u A[9];
    load_round0<NT>(W, n_out, nb, row, A);  // in flight while the activation row is prepared
    if constexpr (FUSE)
        quant_row_to_lds(xf, nb, lds);
    else
        copy_row_to_lds(xq, xd, xs, nb, lds);
    __syncthreads();
    rowgroup_body<NT, NR>(W, n_out, nb, row, lds, A, y);
}

// Up to SYN_BATCH independent single-row GEMVs in one launch: problem p takes workgroups
// [wg_begin[p], wg_begin[p+1]); its activation row was quantized into ws[p] beforehand.  A row
// takes P lanes (P = 16, 32 or 64, the smallest holding all nb <= 64 of its super-blocks), lane
// j its super-block j, so every lane loads exactly one block and no wavefront holds a second
// block's registers: the kernel keeps enough wavefronts resident to cover HBM latency.  Each
// row's terms are folded in order by one lane from LDS.
struct DecBatch {
    const uint8_t* W[SYN_BATCH];
    const uint8_t* ws[SYN_BATCH];  // FUSE = 0: the Q8_K row, quantized beforehand
    const float* x[SYN_BATCH];     // FUSE = 1: the F32 row, quantized by every workgroup
    const uint32_t* active;        // FUSE = 1: a step descriptor's rows_active (0: skip), or null
    float* y[SYN_BATCH];
    int n_out[SYN_BATCH];
    int nb[SYN_BATCH];
    int wg_begin[SYN_BATCH + 1];
    int np;
};

SYN_DEV int lanes_per_row(int nb) { return nb <= 16 ? 16 : nb <= 32 ? 32 : 64; }

// Wavefronts per workgroup of k_gemv_q4k_batch for each weight layout.
template <int LAYOUT>
constexpr int dec_waves() { return LAYOUT == LAYOUT_X8 ? 8 : 4; }

// LAYOUT 0 (the GGUF order): each lane reads its 144-byte super-block with nine 16-byte loads.
// LAYOUT 1 (x8): chunk q of the blocks of eight consecutive super-blocks sits together (see
// layout.hpp), so the nine loads of a wavefront each read whole 128-byte lines, which streams at
// a higher rate with non-temporal loads (the weights are read once).
// FUSE = 1 (X8 weights; a lone Gemv op on an F32 row, one launch): the workgroup loads its
// problem's F32 row into registers before the block's loads, and quantizes it to Q8_K in LDS
// while they fly (crates/kernels-cpu/src/gemv/act.rs:351-373, the same steps as the separate
// quantizer).  Rows of at most 64 super-blocks: two 16-value pieces per thread at 512 threads.
// For a whole layer the separate quantization launch is faster (each workgroup re-quantizing
// its row costs more than the launch it saves).
constexpr int FUSE_PIECES = 2;
// a wavefront's 64 fold terms in LDS, padded by four words so that the rows' 16-byte reads of a
// workgroup fold start in different banks
constexpr int DEC_TS = 68;

// Resident wavefronts per SIMD: 6 (80 registers); the fused form holds the row pieces too
// (4: 128 registers, no spills).
template <int LAYOUT, int FUSE>
constexpr int dec_occupancy() { return FUSE ? 4 : 6; }

// GATED = 1 (GateUpAct{Silu}, one fused launch): the matrix stacks n_out gate rows, then n_out
// up rows; the first half of the wavefronts computes gate rows and the second half the same up
// rows, and y[i] = silu(g_i) * u_i (crates/kernels/src/reference/linear.rs:75-112 with the
// Gemv values, the product rounded once) is formed after one LDS exchange.
// WV: wavefronts per workgroup (dec_waves by default; 16 for the fused form at long rows, where
// every workgroup re-quantizes the row: fewer, larger workgroups quantize it fewer times).
template <int LAYOUT, int FUSE, int GATED, int WV = dec_waves<LAYOUT>()>
__global__ __launch_bounds__(64 * WV)
__attribute__((amdgpu_waves_per_eu(dec_occupancy<LAYOUT, FUSE>())))
void k_gemv_q4k_batch(DecBatch bt) {
    if (active_rows(bt.active, 0, 1) == 0) return;  // a step with no active row
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int WAVES = WV;
    constexpr int RW = GATED ? WAVES / 2 : WAVES;  // wavefronts per set of output rows
    int p = 0;
    while (p + 1 < bt.np && (int)blockIdx.x >= bt.wg_begin[p + 1]) ++p;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint8_t* W = bt.W[p];
    const int n_out = bt.n_out[p], nb = bt.nb[p];
    const int P = lanes_per_row(nb);
    const int rows_per_wave = 64 / P;
    const int row = (((int)blockIdx.x - bt.wg_begin[p]) * RW + wave % RW) * rows_per_wave + lane / P;
    const bool up_half = GATED && wave >= RW;
    const int mrow = up_half ? n_out + row : row;  // the matrix row
    const int b = lane % P;
    const bool ok = row < n_out && b < nb;
    static_assert(!FUSE || LAYOUT == LAYOUT_X8, "the fused form reads X8 weights");
    float xv[FUSE ? FUSE_PIECES : 1][16];
    if constexpr (FUSE) {
        // unconditional loads (pieces past the row re-read its last piece, unused): a load in a
        // branch would make the compiler wait for it before the block's loads below
#pragma unroll
        for (int i = 0; i < FUSE_PIECES; ++i) {
            const int c = (int)threadIdx.x + i * 64 * WAVES;
            load_block16(bt.x[p], c < nb * 16 ? c : nb * 16 - 1, xv[i]);
        }
    } else if constexpr (LAYOUT == LAYOUT_X8) {
        // the activation row streams into LDS first, with no registers held (codes column by
        // column, 16 lanes per column to keep the bank skew; sums and scales contiguous), so the
        // block's loads below queue behind it and the row is in place when they land
        const ActLayout L0 = act_layout(ACT_Q8K, 1, (uint64_t)nb * 256);
        const uint8_t* wsp = bt.ws[p];
        const uint32_t l0 = lds_addr(lds);
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        for (int c = wv; c < nb; c += WAVES)
            if (lane < 16) lds_dma16(16u * (uint32_t)lane, wsp + L0.codes + (size_t)c * 256, l0 + (uint32_t)(c * COL));
        if (wv == 0) {
            for (int u = 0; u * 64 < nb * 2; ++u)
                if (u * 64 + lane < nb * 2)
                    lds_dma16(16u * (uint32_t)lane, wsp + L0.sums + (size_t)u * 1024, l0 + (uint32_t)(xs_off(nb) + u * 1024));
            // the scales' last chunk reads up to 12 bytes past them: workspace padding, and LDS up
            // to the fold terms (which start at the 16-byte-aligned end of the row)
            if (lane * 4 < nb) lds_dma16(16u * (uint32_t)lane, wsp + L0.d, l0 + (uint32_t)xd_off(nb));
        }
    }
    // the lane's block
    v4u A[9];
    if constexpr (LAYOUT == LAYOUT_X8) {
        const uint64_t nblocks = (uint64_t)(GATED ? 2 : 1) * n_out * (uint64_t)nb;
        const uint64_t g = ok ? (uint64_t)mrow * nb + b : 0;
        const uint8_t* src = W + x8_chunk_offset(g, 0, nblocks);
        const uint32_t step = 16u * x8_group_blocks(g, nblocks);
#pragma unroll
        for (int i = 0; i < 9; ++i) A[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + step * i));
    } else {
        const uint8_t* src = ok ? W + (int64_t)mrow * nb * 144 + (int64_t)b * 144 : W;
#pragma unroll
        for (int i = 0; i < 9; ++i) A[i] = *reinterpret_cast<const v4u*>(src + 16 * i);
    }
    if constexpr (FUSE) {
#pragma unroll
        for (int i = 0; i < FUSE_PIECES; ++i) {
            const int c = (int)threadIdx.x + i * 64 * WAVES;
            if (c < nb * 16) quant16_to_lds(xv[i], c, nb, lds);  // 16-lane groups stay whole
        }
        lds_barrier();
    } else if constexpr (LAYOUT == LAYOUT_X8) {
        wait_vm<9>();  // this wavefront's row loads, all older than the block's nine
        lds_barrier();
    } else {
        const ActLayout L = act_layout(ACT_Q8K, 1, (uint64_t)nb * 256);
        copy_row_to_lds(reinterpret_cast<const int8_t*>(bt.ws[p] + L.codes),
                        reinterpret_cast<const float*>(bt.ws[p] + L.d),
                        reinterpret_cast<const int32_t*>(bt.ws[p] + L.sums), nb, lds);
        __syncthreads();
    }
    const float t = q4k_term_lds(A, lds, nb, ok ? b : 0);
    // in-order fold: the row's P terms (+0.0 past its nb blocks, which leaves a sum that
    // started from +0.0 unchanged) added by the row's first lane
    float* terms0 = reinterpret_cast<float*>(lds + align_up(q4k_dec_lds(nb), 16));
    float* terms = terms0 + wave * DEC_TS;
    terms[lane] = ok ? t : 0.0f;
    float acc = 0.0f;
    if (!GATED && P == 64) {  // uniform per workgroup
        // one row a wavefront: the workgroup's rows folded together, lane w of wavefront 0
        // adding wavefront w's terms (one instruction stream for every row, not one per row)
        lds_barrier();
        const int frow = ((int)blockIdx.x - bt.wg_begin[p]) * RW + lane;
        if (wave == 0 && lane < WAVES && frow < n_out) {
            const float4* tv = reinterpret_cast<const float4*>(terms0 + lane * DEC_TS);
            for (int q = 0; q < (nb + 3) / 4; ++q) {
                const float4 v = tv[q];
                acc = acc + v.x;
                acc = acc + v.y;
                acc = acc + v.z;
                acc = acc + v.w;
            }
            bt.y[p][frow] = acc;
        }
        return;
    }
    wave_lds_sync();
    if (b == 0 && row < n_out) {
        const float4* tv = reinterpret_cast<const float4*>(terms + lane);
        for (int q = 0; q < P / 4; ++q) {
            const float4 v = tv[q];
            acc = acc + v.x;
            acc = acc + v.y;
            acc = acc + v.z;
            acc = acc + v.w;
        }
        if constexpr (!GATED) bt.y[p][row] = acc;
    }
    if constexpr (GATED) {
        // the gate sums to the up wavefronts holding the same rows
        float* gsum = terms0 + WAVES * DEC_TS;
        if (!up_half && b == 0) gsum[(wave % RW) * 64 + lane] = acc;
        lds_barrier();
        if (up_half && b == 0 && row < n_out) bt.y[p][row] = ref_silu(gsum[(wave % RW) * 64 + lane]) * acc;
    }
}


// K up to 32768: at most 8 rounds, and the activation row within 41 KB of LDS.
bool q4k_dec_supported(int k) { return k % 256 == 0 && k > 0 && k <= 32768; }

template <int FUSE>
static void launch_dec(const uint8_t* W, int n_out, int nb, const float* xf, const int8_t* xq,
                       const float* xd, const int32_t* xs, float* y, hipStream_t stream,
                       const uint32_t* active = nullptr) {
    const int total_rg = (n_out + 3) / 4;
    const dim3 grid((unsigned)((total_rg + 3) / 4));
    const size_t lds = q4k_dec_lds(nb);
#define SYN_DEC(NR)                                                                         \
    hipLaunchKernelGGL((k_gemv_q4k_dec<FUSE, 0, NR>), grid, dim3(256), lds, stream, W, n_out, nb, \
                       xf, xq, xd, xs, y, active)
    switch ((nb + 15) / 16) {
    case 1: SYN_DEC(1); break;
    case 2: SYN_DEC(2); break;
    case 3: SYN_DEC(3); break;
    case 4: SYN_DEC(4); break;
    case 5: SYN_DEC(5); break;
    case 6: SYN_DEC(6); break;
    case 7: SYN_DEC(7); break;
    default: SYN_DEC(8); break;
    }
#undef SYN_DEC
}

void launch_gemv_q4k_dec_f32(const uint8_t* W, int n_out, int k, const float* x, float* y,
                             hipStream_t stream, const uint32_t* active) {
    launch_dec<1>(W, n_out, k / 256, x, nullptr, nullptr, nullptr, y, stream, active);
}

void launch_gemv_q4k_dec_ws(const uint8_t* W, int n_out, int k, const uint8_t* ws, float* y,
                            hipStream_t stream) {
    const ActLayout L = act_layout(ACT_Q8K, 1, (uint64_t)k);
    launch_dec<0>(W, n_out, k / 256, nullptr, reinterpret_cast<const int8_t*>(ws + L.codes),
                  reinterpret_cast<const float*>(ws + L.d),
                  reinterpret_cast<const int32_t*>(ws + L.sums), y, stream);
}

template <int LAYOUT, int FUSE, int GATED = 0, int WV = dec_waves<LAYOUT>()>
static void launch_batch(int np, const uint8_t* const* W, const int* n_out, const int* k,
                         const uint8_t* const* ws, const float* const* x, float* const* y,
                         hipStream_t stream, const uint32_t* active = nullptr) {
    constexpr int WAVES = WV;
    constexpr int RW = GATED ? WAVES / 2 : WAVES;
    DecBatch bt{};
    bt.np = np;
    bt.active = active;
    int wg = 0, max_nb = 0;
    for (int p = 0; p < np; ++p) {
        bt.W[p] = W[p];
        bt.ws[p] = ws ? ws[p] : nullptr;
        bt.x[p] = x ? x[p] : nullptr;
        bt.y[p] = y[p];
        bt.n_out[p] = n_out[p];
        bt.nb[p] = k[p] / 256;
        bt.wg_begin[p] = wg;
        const int nb = bt.nb[p];
        const int rows_per_wg = RW * (64 / (nb <= 16 ? 16 : nb <= 32 ? 32 : 64));
        wg += (n_out[p] + rows_per_wg - 1) / rows_per_wg;
        if (nb > max_nb) max_nb = nb;
    }
    bt.wg_begin[np] = wg;
    if (wg == 0) return;
    // the activation row, then the fold terms per wavefront (and the gate sums when GATED)
    hipLaunchKernelGGL((k_gemv_q4k_batch<LAYOUT, FUSE, GATED, WV>), dim3(wg), dim3(64 * WAVES),
                       align_up(q4k_dec_lds(max_nb), 16) + (GATED ? 2 : 1) * WAVES * DEC_TS * 4, stream, bt);
}

void launch_gemv_q4k_batch(int layout, int np, const uint8_t* const* W, const int* n_out, const int* k,
                           const uint8_t* const* ws, float* const* y, hipStream_t stream) {
    if (layout == LAYOUT_X8)
        launch_batch<LAYOUT_X8, 0>(np, W, n_out, k, ws, nullptr, y, stream);
    else
        launch_batch<LAYOUT_SOURCE, 0>(np, W, n_out, k, ws, nullptr, y, stream);
}

bool gemv_q4k_batch_fusable(int k) { return k % 256 == 0 && k > 0 && k <= 64 * 256; }

void launch_gemv_q4k_batch_f32(const uint8_t* const* W, int np, const int* n_out, const int* k,
                               const float* const* x, float* const* y, hipStream_t stream,
                               const uint32_t* active) {
    int max_k = 0, wg8 = 0;  // wg8: workgroups at eight wavefronts
    for (int p = 0; p < np; ++p) {
        max_k = k[p] > max_k ? k[p] : max_k;
        const int nb = k[p] / 256, rows_per_wg = 8 * (64 / (nb <= 16 ? 16 : nb <= 32 ? 32 : 64));
        wg8 += (n_out[p] + rows_per_wg - 1) / rows_per_wg;
    }
    if (max_k > 32 * 256)  // rows of more than 32 super-blocks: 16-wavefront workgroups
        launch_batch<LAYOUT_X8, 1, 0, 16>(np, W, n_out, k, nullptr, x, y, stream, active);
    else if (wg8 <= 128)  // at most half the CUs busy: 4-wavefront workgroups, twice as many
        launch_batch<LAYOUT_X8, 1, 0, 4>(np, W, n_out, k, nullptr, x, y, stream, active);
    else
        launch_batch<LAYOUT_X8, 1>(np, W, n_out, k, nullptr, x, y, stream, active);
}

void launch_gate_up_q4k_f32(const uint8_t* W, int n, int k, const float* x, float* y, hipStream_t stream,
                            const uint32_t* active) {
    launch_batch<LAYOUT_X8, 1, 1>(1, &W, &n, &k, nullptr, &x, &y, stream, active);
}

// ---- the x8 repack: a permutation of whole 16-byte chunks --------------------------------------
// Two to four rows over X8 weights: the one-row decode kernel's loads and its one block per
// lane, with the NR activation rows (Q8_K, quantized beforehand) side by side in LDS, so the
// weights stream once and each lane computes its block's term against every row; the terms of
// each (weight row, activation row) pair of a wavefront are folded in block order by a lane of
// their own, one stream of adds for all the pairs.  Rows of up to 64 super-blocks; rows past the
// step's active rows are neither computed nor written.  FUSE = 1 (rows of at most 16
// super-blocks): the workgroup quantizes the F32 rows to Q8_K in LDS itself, as the one-row
// kernel does, the rows' loads issued before the block's: one launch (two rows, 14336 x 4096:
// 10.2 against 10.7 us; 4096 x 4096: 6.4 against 7.8 us, before the shared fold).
constexpr int XR_WAVES = 8;
constexpr int XR_TS = XR_WAVES * 64 + 4;  // one activation row's terms in LDS, padded

SYN_HD inline size_t xr_row_lds(int nb) { return align_up(q4k_dec_lds(nb) + 16, 16); }  // + the scales' 16-byte tail

template <int NR, int FUSE>
__global__ __launch_bounds__(64 * XR_WAVES) void k_gemv_q4k_x8_rows(const uint8_t* __restrict__ W, int n_out, int nb,
                                                                  const uint8_t* __restrict__ ws, int rows_ws, int rows,
                                                                  const float* __restrict__ x,
                                                                  float* __restrict__ y,
                                                                  const uint32_t* __restrict__ active) {
    rows = active_rows(active, 0, rows);
    if (rows == 0) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int P = lanes_per_row(nb);
    const int row = ((int)blockIdx.x * XR_WAVES + wave) * (64 / P) + lane / P;
    const int b = lane % P;
    const bool ok = row < n_out && b < nb;
    const int RB = (int)xr_row_lds(nb);
    // FUSE: 16-value pieces of the rows (task = row * 16 nb + piece), loaded unconditionally (a
    // task past the last re-reads it, unused) before the block's loads
    constexpr int PIECES = FUSE ? (NR * 256 + 64 * XR_WAVES - 1) / (64 * XR_WAVES) : 1;
    float xv[PIECES][16];
    if constexpr (FUSE) {
        const int ntask = NR * nb * 16;
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int tk0 = (int)threadIdx.x + i * 64 * XR_WAVES, tk = tk0 < ntask ? tk0 : ntask - 1;
            const int r = tk / (nb * 16);
            load_block16(x + (int64_t)r * nb * 256, tk - r * nb * 16, xv[i]);
        }
    }
    // the activation rows stream into LDS first (as the one-row kernel's), then the block
    const ActLayout L = act_layout(ACT_Q8K, (uint64_t)rows_ws, (uint64_t)nb * 256);
    const uint32_t l0 = lds_addr(lds);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (FUSE || r >= rows) break;  // uniform
        const uint8_t* codes = ws + L.codes + (size_t)r * nb * 256;
        const uint32_t lr = l0 + (uint32_t)(r * RB);
        for (int c = wv; c < nb; c += XR_WAVES)
            if (lane < 16) lds_dma16(16u * (uint32_t)lane, codes + (size_t)c * 256, lr + (uint32_t)(c * COL));
        if (wv == 0) {
            const uint8_t* sums = ws + L.sums + (size_t)r * nb * 32;
            for (int u = 0; u * 64 < nb * 2; ++u)
                if (u * 64 + lane < nb * 2)
                    lds_dma16(16u * (uint32_t)lane, sums + (size_t)u * 1024, lr + (uint32_t)(xs_off(nb) + u * 1024));
            // up to 12 bytes past the row's scales: the next row's, or the sums after them
            if (lane * 4 < nb) lds_dma16(16u * (uint32_t)lane, ws + L.d + (size_t)r * nb * 4, lr + (uint32_t)xd_off(nb));
        }
    }
    v4u A[9];
    {
        const uint64_t nblocks = (uint64_t)n_out * (uint64_t)nb;
        const uint64_t g = ok ? (uint64_t)row * nb + b : 0;
        const uint8_t* src = W + x8_chunk_offset(g, 0, nblocks);
        const uint32_t step = 16u * x8_group_blocks(g, nblocks);
#pragma unroll
        for (int i = 0; i < 9; ++i) A[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + step * i));
    }
    if constexpr (FUSE) {
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int tk = (int)threadIdx.x + i * 64 * XR_WAVES, r = tk / (nb * 16);
            if (r < NR && r < rows) quant16_to_lds(xv[i], tk - r * nb * 16, nb, lds + r * RB);  // 16-lane groups stay whole
        }
        lds_barrier();
    } else {
        wait_vm<9>();  // this wavefront's row loads, all older than the block's nine
        lds_barrier();
    }
    // terms [activation row r][wavefront][lane], a row's set padded by four words
    float* terms = reinterpret_cast<float*>(lds + (size_t)NR * RB);
    float t[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) t[r] = r < rows ? q4k_term_lds(A, lds + r * RB, nb, ok ? b : 0) : 0.0f;
#pragma unroll
    for (int r = 0; r < NR; ++r) terms[r * XR_TS + wave * 64 + lane] = ok ? t[r] : 0.0f;
    wave_lds_sync();
    // lane j + rpw r folds the wavefront's weight row j against activation row r: one stream of
    // P adds for every (row, activation row) pair of the wavefront
    const int rpw = 64 / P, fr = lane % rpw, ar = lane / rpw;
    const int frow = ((int)blockIdx.x * XR_WAVES + wave) * rpw + fr;
    if (ar < rows && ar < NR && frow < n_out) {
        const float4* tv = reinterpret_cast<const float4*>(terms + ar * XR_TS + wave * 64 + fr * P);
        float acc = 0.0f;
        for (int q = 0; q < P / 4; ++q) {
            const float4 v = tv[q];
            acc = acc + v.x;
            acc = acc + v.y;
            acc = acc + v.z;
            acc = acc + v.w;
        }
        y[(int64_t)ar * n_out + frow] = acc;
    }
}

// Where it is the faster form (measured against the line-order expert kernel over X8 runs,
// 14336 x 4096, 6144 x 4096, 4096 x 4096 and 4096 x 14336): two rows of up to 64 super-blocks
// (9.35 against 13.2 us at 14336 x 4096, level elsewhere); three and four rows of at most 16
// super-blocks in the fused form (14336, 6144 and 4096 rows of 4096: three rows 11.1, 6.8 and
// 6.5 us against 12.0, 7.5 and 7.1 before the shared fold; four rows 13.1, 8.1 and 7.8 against
// 13.2, 8.8 and 7.8 for the expert kernel).
bool gemv_q4k_x8_rows_pick(int n_out, int k, int rows) {
    if (k % 256 || k <= 0 || k > 64 * 256) return false;
    const int nb = k / 256;
    (void)n_out;
    return rows == 2 || ((rows == 3 || rows == 4) && nb <= 16);
}

bool gemv_q4k_x8_rows_fused(int k, int rows) { return rows >= 2 && rows <= 4 && k % 256 == 0 && k > 0 && k <= 16 * 256; }

void launch_gemv_q4k_x8_rows(const uint8_t* W, int n_out, int k, const uint8_t* ws, const float* x, int rows,
                             float* y, hipStream_t stream, const uint32_t* active) {
    const int nb = k / 256;
    const int rows_per_wg = XR_WAVES * (64 / (nb <= 16 ? 16 : nb <= 32 ? 32 : 64));
    const dim3 grid((unsigned)((n_out + rows_per_wg - 1) / rows_per_wg));
#define SYN_XR(NR, FUSE)                                                                                    \
    do {                                                                                                     \
        const size_t lds = (size_t)NR * xr_row_lds(nb) + (size_t)NR * XR_TS * 4;                             \
        static const hipError_t lds_ok = hipFuncSetAttribute((const void*)k_gemv_q4k_x8_rows<NR, FUSE>,       \
                                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024); \
        (void)lds_ok; /* a refusal shows as the launch's error */                                            \
        hipLaunchKernelGGL((k_gemv_q4k_x8_rows<NR, FUSE>), grid, dim3(64 * XR_WAVES), lds, stream, W, n_out, nb, ws, \
                           rows, rows, x, y, active);                                                        \
    } while (0)
    if (x) {  // the rows quantized in the workgroups (gemv_q4k_x8_rows_fused)
        if (rows <= 2)
            SYN_XR(2, 1);
        else if (rows == 3)
            SYN_XR(3, 1);
        else
            SYN_XR(4, 1);
    } else if (rows <= 2) {
        SYN_XR(2, 0);
    } else if (rows == 3) {
        SYN_XR(3, 0);
    } else {
        SYN_XR(4, 0);
    }
#undef SYN_XR
}

__global__ __launch_bounds__(256) void k_q4k_x8(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                uint64_t nblocks, int inverse) {
    const uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // source chunk (GGUF order)
    if (c >= nblocks * 9) return;
    const uint64_t g = c / 9, q = c - g * 9;
    const uint64_t to = x8_chunk_offset(g, (int)q, nblocks);
    const uint64_t from = c * 16;
    const v4u v = *reinterpret_cast<const v4u*>(src + (inverse ? to : from));
    *reinterpret_cast<v4u*>(dst + (inverse ? from : to)) = v;
}

void launch_q4k_x8(const uint8_t* src, uint8_t* dst, uint64_t nblocks, int inverse, hipStream_t stream) {
    const uint64_t chunks = nblocks * 9;
    if (chunks == 0) return;
    hipLaunchKernelGGL(k_q4k_x8, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, src, dst, nblocks,
                       inverse);
}

}  // namespace syn
