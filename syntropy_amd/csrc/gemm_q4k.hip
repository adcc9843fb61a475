// Prefill Q4_K GEMM on the gfx950 matrix cores: Y[t][n] for many activation rows t, each
// output the exact Gemv value (crates/kernels-cpu/src/gemv.rs:435-547: per super-block the
// term (d*dx)*S1 - (dmin*dx)*S2 with S1 = sum_j sc_j D_j and S2 = sum_j m_j s_j exact, folded
// in super-block order from +0.0).  The reference's Gemm is the same value (its Gemm kind is
// Gemv at a larger bucket, crates/kernels/src/reference/linear.rs:11-13).
//
// Exact sums on F16 matrix cores.  v_mfma_f32_16x16x32_f16 multiplies F16 operands exactly and
// accumulates in F32; when every operand is an integer and every partial sum stays below 2^24
// in magnitude, the F32 result is the exact integer whatever the order of the additions.  Per
// super-block the kernel feeds, for k = 0..255:
//   A[t][k] = x code (Q8_K, |x| <= 127, written as F16 by k_gemm_act);
//   B[k][n] = sc_j(k) * q_k - 512   (|B| <= 512, exact F16: the 6-bit scale folded into the
//                                     4-bit code, offset so that 256 * 127 * 512 < 2^24)
// so one accumulator holds D = S1 - 512 X exactly, X = sum_k x_k (a per-token integer the
// activation kernel stores), and fma(512, X, D) = fl(S1): one rounding of the exact S1, which
// is the reference's `S1 as f32`.  S2 comes from a second product per tile: A = (l_j, 64 h_j)
// with s_j = 64 h_j + l_j, B = (m_j, m_j), also exact.  The term and the fold are plain F32
// operations in the reference's order.
//
// B from the packed nibbles, two codes per instruction: the code dword (or it shifted right by
// 8) masked to the low nibbles of its 16-bit halves and ORed with 0x6400 in each half is the
// F16 pair (1024 + q0, 1024 + q1), and one v_pk_fma_f16 with (sc, -(1024 sc + 512)) gives
// sc*q - 512; masked to the high nibbles it is (1024 + 16 q0, 1024 + 16 q1), and the FMA takes
// (sc/16, -(64 sc + 512)).  Both are exact: every constant is an exact F16 (1024 sc + 512 =
// 512 (2 sc + 1)) and the FMA rounds once, to an exact integer.  The k order inside
// a super-block is free (the sum is exact), so each lane's eight k slots of an instruction are
// the codes of four consecutive bytes, low nibbles then high: k_gemm_act writes the activations
// in the same order.
//
// Tiling.  A workgroup computes 64 tokens x 256 rows; each of its 8 wavefronts 64 tokens x 32
// rows as 4 x 2 tiles of 16 x 16 (two wavefronts per SIMD hide each other's LDS and matrix-core
// latencies), so each A operand serves two row tiles and each B operand four token tiles.  Per super-block the weight rows (144 bytes each), the 64 tokens' codes and their
// sums, scales and X stream from global memory into LDS with global_load_lds_dwordx4 (no
// registers held while they fly), one stage ahead, in a ring of two 72 KB stages.
#include <type_traits>
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// ============================================================================================
// Activation layout (GemmAct)
// ============================================================================================
//
// For tpad = T rounded up to 64 and nb = k / 256 super-blocks:
//   codes [nb][tpad][256] F16: chunk c = 8p + s (8 codes) of token t holds the values
//         64p + 4s + {0, 2, 1, 3, 32, 34, 33, 35} and sits at chunk position c ^ (t & 15), so the
//         16 lanes of a read touch 16 distinct 16-byte bank groups;
//   tail  [nb][ s2: tpad x 16 F16 | dx: tpad x F32 | X: tpad x F32 ]: s2 = (l_0..l_7,
//         64 h_0..64 h_7) with s_j = 64 h_j + l_j, 0 <= l_j < 64; dx the Q8_K scale; X the sum
//         of the block's 256 codes.
// Rows t >= T are zero.
constexpr int GM_TAIL_ROW = 40;  // tail bytes per token per super-block

size_t gemm_act_bytes(int64_t tpad, int k) {
    const int64_t nb = k / 256;
    return align_up((uint64_t)(nb * tpad * 512), 256) + align_up((uint64_t)(nb * tpad * GM_TAIL_ROW), 256);
}

GemmAct gemm_act_at(uint8_t* base, int64_t tpad, int k) {
    const int64_t nb = k / 256;
    GemmAct a;
    a.codes = base;
    a.tail = base + align_up((uint64_t)(nb * tpad * 512), 256);
    a.tpad = (int)tpad;
    return a;
}

// One wavefront per (super-block b, token t): the Q8_K block of crates/kernels-cpu/src/gemv/
// act.rs:351-373 (q8k_block_lane), written in the GEMM order.  Lane l holds values 4l..4l+3
// (v4, loaded by the caller): sub-block j = l / 8, k part p = l / 16, nibble half h = (l / 8) & 1,
// dword s = l & 7.  A padding position (live false) writes zeros.
SYN_DEV void gemm_act_block(float4 v4, bool live, int b, int t, GemmAct a, int lane) {
    uint32_t q = 0;
    int sum32 = 0, xsum = 0;
    float d = 0.0f;
    if (live) {  // uniform over the wavefront
        const Q8KLane r = q8k_block_lane(v4, lane);
        q = r.packed;
        sum32 = r.sum32;
        d = r.d;
        xsum = sum32;
        xsum += __shfl_xor(xsum, 8);
        xsum += __shfl_xor(xsum, 16);
        xsum += __shfl_xor(xsum, 32);
    }
    const int p = lane >> 4, h = (lane >> 3) & 1, s = lane & 7;
    auto code = [&](int i) { return (_Float16)(float)(int8_t)(q >> (8 * i)); };
    h2 lo = {code(0), code(2)}, hi = {code(1), code(3)};
    const int pos = (8 * p + s) ^ (t & 15);
    uint8_t* dst = a.codes + ((int64_t)b * a.tpad + t) * 512 + pos * 16 + 8 * h;
    uint2 v;
    v.x = __builtin_bit_cast(uint32_t, lo);
    v.y = __builtin_bit_cast(uint32_t, hi);
    *reinterpret_cast<uint2*>(dst) = v;
    uint8_t* tail = a.tail + (int64_t)b * a.tpad * GM_TAIL_ROW;
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        const int hj = sum32 >> 6;  // floor: s = 64 h + l with 0 <= l < 64
        const int lj = sum32 - 64 * hj;
        _Float16* s2 = reinterpret_cast<_Float16*>(tail + (int64_t)t * 32);
        s2[j] = (_Float16)(float)lj;
        s2[8 + j] = (_Float16)(float)(64 * hj);
    }
    if (lane == 0) {
        reinterpret_cast<float*>(tail + (int64_t)a.tpad * 32)[t] = d;
        reinterpret_cast<float*>(tail + (int64_t)a.tpad * 36)[t] = (float)xsum;
    }
}

// A wavefront takes BPW consecutive super-blocks of one row, their loads issued together before
// any is quantized: at many blocks (ACT_WIDE_ITEMS or more) four a wavefront, which keeps more
// bytes in flight per wavefront (14336-wide rows at 2048 tokens: 45 against 50 us; the MoE layer's
// h: 43 against 56 us); below that one, which keeps more wavefronts (4096-wide: 15 against
// 17 us).  Item = (block group g, position t), t fastest.
constexpr int64_t ACT_WIDE_ITEMS = 65536;

template <int BPW, class RowOf>
SYN_DEV void gemm_act_blocks(int nb, int64_t item, GemmAct a, int lane, RowOf row_of) {
    const int ng = (nb + BPW - 1) / BPW;
    if (item >= (int64_t)ng * a.tpad) return;
    const int g = (int)(item / a.tpad), t = (int)(item - (int64_t)g * a.tpad);
    const float* row = row_of(t);  // null: a padding position
    float4 v[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const int b = g * BPW + j;
        v[j] = row && b < nb ? reinterpret_cast<const float4*>(row + (int64_t)b * 256)[lane] : float4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const int b = g * BPW + j;
        if (b < nb) gemm_act_block(v[j], row != nullptr, b, t, a, lane);  // uniform
    }
}

// Blocks a wavefront for nb super-blocks at tpad positions, and the wavefronts that takes.
SYN_HD inline int gemm_act_bpw(int nb, int64_t tpad) { return (int64_t)nb * tpad >= ACT_WIDE_ITEMS ? 4 : 1; }
SYN_HD inline int64_t gemm_act_items(int nb, int64_t tpad) {
    const int bpw = gemm_act_bpw(nb, tpad);
    return (int64_t)((nb + bpw - 1) / bpw) * tpad;
}

template <int BPW>
__global__ __launch_bounds__(256) void k_gemm_act(const float* __restrict__ x, int T, int k, GemmAct a,
                                                  const uint32_t* __restrict__ active) {
    T = active_rows(active, 0, T);  // inactive rows are written as padding
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    gemm_act_blocks<BPW>(k / 256, item, a, lane, [&](int t) { return t < T ? x + (int64_t)t * k : nullptr; });
}

void launch_gemm_act(const float* x, int T, int k, GemmAct a, hipStream_t stream, const uint32_t* active) {
    const int64_t items = gemm_act_items(k / 256, a.tpad);
    if (items == 0) return;
    const dim3 grid((unsigned)((items + 3) / 4));
    if (gemm_act_bpw(k / 256, a.tpad) == 4)
        hipLaunchKernelGGL(k_gemm_act<4>, grid, dim3(256), 0, stream, x, T, k, a, active);
    else
        hipLaunchKernelGGL(k_gemm_act<1>, grid, dim3(256), 0, stream, x, T, k, a, active);
}

// ============================================================================================
// The GEMM
// ============================================================================================

constexpr int GM_TT = 64;                           // tokens per workgroup
constexpr int GM_WAVES = 8;                         // wavefronts per workgroup
constexpr int GM_NT = 2;                            // 16-row tiles per wavefront
constexpr int GM_MT = 4;                            // 16-token tiles per wavefront
constexpr int GM_ROWS = GM_WAVES * 16 * GM_NT;      // rows per workgroup
constexpr int GM_WB = GM_ROWS * 144;                // weight bytes per stage
constexpr int GM_AB = GM_TT * 512;                  // code bytes per stage
constexpr int GM_TB = GM_TT * GM_TAIL_ROW;          // s2 | dx | X bytes per stage
constexpr int GM_WSLOT = GM_WB / 1024;              // wavefront loads (64 x 16 bytes) of each part
constexpr int GM_ASLOT = GM_AB / 1024;
constexpr int GM_TSLOT = (GM_TB + 1023) / 1024;
constexpr int GM_WPW = (GM_WSLOT + GM_WAVES - 1) / GM_WAVES;  // weight slots per wavefront (at most)
constexpr int GM_PER_WAVE = GM_WPW + GM_ASLOT / GM_WAVES + 1;
static_assert(GM_ASLOT % GM_WAVES == 0 && GM_TSLOT <= GM_WAVES, "slot split");
static_assert(GM_WB % 1024 == 0 && GM_AB % 1024 == 0, "wavefront-sized weight and code parts");

struct GemmArgs {
    const uint8_t* W;
    int layout;  // LAYOUT_SOURCE, LAYOUT_X8 (rows of whole 8-block runs) or LAYOUT_TILE64 (the experts)
    const uint8_t* codes;
    const uint8_t* tail;
    float* y;
    int N, T, nb, tpad;
    uint32_t rb;  // weight row bytes
    const uint32_t* active;  // a step descriptor's rows_active, or null
};

// The lane's 32-bit offsets of its loads of one stage, relative to the part's base of the
// super-block (weights: W + 144 b; codes: codes + (b tpad + t0) 512; tail: tail + b tpad 40).
struct GemmSlots {
    uint32_t woff[GM_WPW];
    uint32_t toff;
    int nw, nt;     // weight and tail slots of this wavefront (uniform)
    bool ton;       // this lane's tail chunk exists
};

SYN_DEV GemmSlots gemm_slots(const GemmArgs& g, int wave, int lane, int n0, int t0) {
    GemmSlots s;
    s.nw = 0;
#pragma unroll
    for (int u = 0; u < GM_WPW; ++u) {
        const int gs = wave + GM_WAVES * u;
        const int ci = 64 * gs + lane, row = ci / 9, part = ci - 9 * (ci / 9);
        const int r = n0 + row < g.N ? n0 + row : g.N - 1;
        // chunk `part` of the row's block: 16 bytes on in GGUF order and TILE64, 128 (a run's chunk
        // row) in X8
        s.woff[u] = g.layout == LAYOUT_TILE64 ? (uint32_t)tile64_row_offset((uint32_t)r, g.rb) + 16u * (uint32_t)part
                                               : (uint32_t)r * g.rb + (g.layout == LAYOUT_X8 ? 128u : 16u) * (uint32_t)part;
        if (gs < GM_WSLOT) s.nw = u + 1;
    }
    // tail slot: wave w takes tail part w if it exists
    s.nt = wave < GM_TSLOT ? 1 : 0;
    const int ti = 64 * wave + lane;
    s.ton = s.nt && ti < GM_TB / 16;
    if (ti < GM_TT * 2)
        s.toff = (uint32_t)t0 * 32u + 16u * (uint32_t)ti;
    else if (ti < GM_TT * 2 + GM_TT / 4)
        s.toff = (uint32_t)g.tpad * 32u + (uint32_t)t0 * 4u + 16u * (uint32_t)(ti - GM_TT * 2);
    else
        s.toff = (uint32_t)g.tpad * 36u + (uint32_t)t0 * 4u + 16u * (uint32_t)(ti - GM_TT * 2 - GM_TT / 4);
    return s;
}


// Issues the wavefront's loads of super-block b: weights and codes into `stage`, the tail into
// `tail`.  Slot order: weight parts wave, wave + 8, ..; code parts wave, wave + 8, ..; tail part
// `wave`.
SYN_DEV void gemm_issue(const GemmArgs& g, const GemmSlots& s, int wave, int lane, int b, int t0,
                        uint8_t* stage, uint8_t* tail) {
    // super-block b of row 0: in X8 block b sits in run b / 8 at position b % 8
    const uint8_t* wb = g.layout == LAYOUT_X8 ? g.W + 1152 * (size_t)(b >> 3) + 16 * (size_t)(b & 7)
                                                  : g.W + 144 * (size_t)b;
    const uint8_t* ab = g.codes + ((size_t)b * g.tpad + t0) * 512;
    const uint8_t* tb = g.tail + (size_t)b * g.tpad * GM_TAIL_ROW;
    const uint32_t st = lds_addr(stage);
#pragma unroll
    for (int u = 0; u < GM_WPW; ++u)
        if (u < s.nw) lds_dma16(s.woff[u], wb, st + 1024u * (uint32_t)(wave + GM_WAVES * u));
#pragma unroll
    for (int u = 0; u < GM_ASLOT / GM_WAVES; ++u) {
        const int gs = wave + GM_WAVES * u;
        lds_dma16(16u * (uint32_t)lane, ab + 1024 * gs, st + (uint32_t)GM_WB + 1024u * (uint32_t)gs);
    }
    if (s.ton) lds_dma16(s.toff, tb, lds_addr(tail) + 1024u * (uint32_t)wave);
}

// The F16 pair (1024 + 16 q0, 1024 + 16 q1) etc. from the nibbles under `mask`.
// (v & mask) | 0x64006400 is one v_bitop3_b32 (truth table 0xEA = (a & b) | c); written as two
// operations the compiler issues an AND and an OR.
SYN_DEV h2 magic_pair(uint32_t v, uint32_t mask) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_bitop3_b32(v, mask, 0x64006400u, 0xEA));
}

SYN_DEV h2 bcast(_Float16 v) { return h2{v, v}; }

// What the fold of a super-block needs from its row headers: d, dmin and the S2 operand.
struct GemmHdr {
    float dd[GM_NT], dm[GM_NT];
    v8h bm[GM_NT];
};

// The matrix-core part of one super-block of the wavefront's 64 tokens x 32 rows, from the
// weights and codes of the stage in LDS: dacc = S1 - 512 X exactly, and the row headers.  Only
// the first NMT 16-token tiles are computed (a tile of fewer entries leaves the rest empty).
template <int NMT>
SYN_DEV void gemm_mfma(const uint8_t* st, int wave, int lane, v4f (&dacc)[GM_MT][GM_NT], GemmHdr& h) {
    const int c = lane & 15, p = lane >> 4;
    const uint8_t* wt = st + (16 * GM_NT * wave) * 144;
    const uint8_t* at = st + GM_WB;
    float (&dd)[GM_NT] = h.dd;
    float (&dm)[GM_NT] = h.dm;
    v8h (&bm)[GM_NT] = h.bm;
    h2 ka[GM_NT], kb[GM_NT];  // (sc, -(1024 sc + 512)) of sub-block 2p, (sc/16, -(64 sc + 512)) of 2p + 1
#pragma unroll
    for (int nt = 0; nt < GM_NT; ++nt) {
        const v4u hdr = *reinterpret_cast<const v4u*>(wt + (16 * nt + c) * 144);
        dd[nt] = f16_to_f32(hdr.x);
        dm[nt] = f16_to_f32(hdr.x >> 16);
        // get_scale_min_k4 (gemv.rs:528-537) on packed bytes
        const uint32_t w0 = hdr.y, w1 = hdr.z, w2 = hdr.w;
        const uint32_t sc_lo = w0 & 0x3F3F3F3Fu;                                 // sc_0..3
        const uint32_t sc_hi = (w2 & 0x0F0F0F0Fu) | ((w0 >> 2) & 0x30303030u);   // sc_4..7
        const uint32_t mn_lo = w1 & 0x3F3F3F3Fu;                                 // m_0..3
        const uint32_t mn_hi = ((w2 >> 4) & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);  // m_4..7
        // this lane group's sub-blocks: 2p (low nibbles) and 2p + 1 (high nibbles)
        const uint32_t scw = p < 2 ? sc_lo : sc_hi;
        const int sa = (int)((scw >> (16 * (p & 1))) & 0xFFu), sb = (int)((scw >> (16 * (p & 1) + 8)) & 0xFFu);
        const float fa = (float)sa, fb = (float)sb;
        ka[nt] = h2{(_Float16)fa, (_Float16)(-(1024.0f * fa + 512.0f))};
        kb[nt] = h2{(_Float16)(fb * 0.0625f), (_Float16)(-(64.0f * fb + 512.0f))};
        // S2 operand: m_0..m_7 in lane groups 0 and 1 (against l_j and 64 h_j), zero in 2 and 3
        const _Float16 on = p < 2 ? (_Float16)1.0f : (_Float16)0.0f;
        const h2 k1 = bcast(on), k0 = bcast((_Float16)(-1024.0f) * on);
        // bytes b0, b1 of a word into the low bits of two halves
        const h2 m01 = __builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, mn_lo, 0x0c010c00u) | 0x64006400u), k1, k0);
        const h2 m23 = __builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, mn_lo, 0x0c030c02u) | 0x64006400u), k1, k0);
        const h2 m45 = __builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, mn_hi, 0x0c010c00u) | 0x64006400u), k1, k0);
        const h2 m67 = __builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, mn_hi, 0x0c030c02u) | 0x64006400u), k1, k0);
        bm[nt] = v8h{m01.x, m01.y, m23.x, m23.y, m45.x, m45.y, m67.x, m67.y};
    }

#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) dacc[mt][nt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int s = 0; s < 8; ++s) {
        v8h bq[GM_NT];
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) {
            // bytes 32p + 4s .. +3 of the row's codes: sub-block 2p (low) and 2p + 1 (high)
            const uint32_t v = *reinterpret_cast<const uint32_t*>(wt + (16 * nt + c) * 144 + 16 + 32 * p + 4 * s);
            // (b0, b2) low nibbles, (b1, b3) low, (b0, b2) high, (b1, b3) high
            const h2 y3 = __builtin_elementwise_fma(magic_pair(v, 0x000F000Fu), bcast(ka[nt].x), bcast(ka[nt].y));
            const h2 y2 = __builtin_elementwise_fma(magic_pair(v >> 8, 0x000F000Fu), bcast(ka[nt].x), bcast(ka[nt].y));
            const h2 y1 = __builtin_elementwise_fma(magic_pair(v, 0x00F000F0u), bcast(kb[nt].x), bcast(kb[nt].y));
            const h2 y4 = __builtin_elementwise_fma(magic_pair(v >> 8, 0x00F000F0u), bcast(kb[nt].x), bcast(kb[nt].y));
            bq[nt] = v8h{y3.x, y3.y, y2.x, y2.y, y1.x, y1.y, y4.x, y4.y};
        }
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) {
            const int t = 16 * mt + c;
            const v8h a = *reinterpret_cast<const v8h*>(at + t * 512 + (((8 * p + s) ^ c) << 4));
#pragma unroll
            for (int nt = 0; nt < GM_NT; ++nt)
                dacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[nt], dacc[mt][nt], 0, 0, 0);
        }
    }
}

// S2 from the tail's code sums, then the super-block's terms folded into the accumulators in
// the reference's rounding order.
template <int NMT>
SYN_DEV void gemm_fold(const uint8_t* tl, int lane, const v4f (&dacc)[GM_MT][GM_NT], const GemmHdr& h,
                       v4f (&acc)[GM_MT][GM_NT]) {
    const int c = lane & 15, p = lane >> 4;
    const v8h zero8 = {};
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
        const v8h as = p < 2 ? *reinterpret_cast<const v8h*>(tl + (16 * mt + c) * 32 + 16 * p) : zero8;
        const v4f dx = *reinterpret_cast<const v4f*>(tl + GM_TT * 32 + (16 * mt + 4 * p) * 4);
        const v4f xs = *reinterpret_cast<const v4f*>(tl + GM_TT * 36 + (16 * mt + 4 * p) * 4);
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) {
            const v4f s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, h.bm[nt], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s1 = __builtin_fmaf(512.0f, xs[i], dacc[mt][nt][i]);  // fl(S1), exact operands
                const float a1 = (h.dd[nt] * dx[i]) * s1;
                const float a2 = (h.dm[nt] * dx[i]) * s2[i];
                acc[mt][nt][i] = acc[mt][nt][i] + (a1 - a2);
            }
        }
    }
}

// The GEMMs' LDS: two stages of weights and codes, then a three-slot ring of tails, so that
// super-block b's fold can run after b + 1's matrix products (its weights and codes are
// overwritten by then; its tail is not until b + 3 is issued).
constexpr int GM_WA = GM_WB + GM_AB;
constexpr int GM_LOOP_LDS = 2 * GM_WA + 3 * GM_TB;
static_assert(GM_WA % 16 == 0 && GM_TB % 16 == 0 && GM_LOOP_LDS <= 160 * 1024, "GEMM LDS");

// The super-block loop of both GEMM kernels.  `issue(b, stage, tail)` issues the wavefront's
// loads of super-block b.  Super-block b's products run first, then b - 1's fold (independent
// work the wavefront can issue between the products), with the two sets of exact sums
// alternating by parity.  Super-block 0 has no fold before it, so it is peeled: the loop's
// products and fold are one straight run of code the scheduler can interleave.  Two schedules
// of the loads, each a super-block ahead of the products:
//   AHEAD: two barriers a super-block; once every wavefront has left b's stage, b + 2's loads go
//     to it at the end of b's step, before the wait for b + 1's, so both may be in flight (the
//     dense GEMM: 425-434 against 438-444 us a launch at 2048 tokens);
//   otherwise one barrier a super-block; once every wavefront's loads of b have landed and every
//     wavefront has left b - 1's products and b - 2's fold, b + 1's loads go to b - 1's stage
//     and b - 2's tail slot (the MoE layer at 2048 tokens: 1.56 against 1.60 ms).
// On return every wavefront is done with the two stages (the caller may reuse them); the tail
// ring may still be read.
template <int NMT, bool AHEAD, class Issue>
SYN_DEV void gemm_loop(int nb, int live, uint8_t* smem, int wave, int lane, Issue&& issue,
                       v4f (&acc)[GM_MT][GM_NT]) {
    uint8_t* tails = smem + 2 * GM_WA;
    issue(0, smem, tails);
    if (AHEAD && nb > 1) issue(1, smem + GM_WA, tails + GM_TB);
    v4f d0[GM_MT][GM_NT], d1[GM_MT][GM_NT];
    GemmHdr h0, h1;
    int slot = 0;  // tail ring slot of b
    auto step = [&](auto fold, int b, v4f (&dc)[GM_MT][GM_NT], GemmHdr& hc, const v4f (&dp)[GM_MT][GM_NT],
                    const GemmHdr& hp) __attribute__((always_inline)) {
        const int prev = slot == 0 ? 2 : slot - 1;  // the slot of b - 1 (b + 2's after the fold)
        const int next = slot == 2 ? 0 : slot + 1;  // the slot of b + 1 (b - 2's)
        if constexpr (AHEAD) {
            wait_vm_n<GM_PER_WAVE>(b + 1 < nb ? live : 0);  // at most b + 1's loads in flight
        } else {
            wait_vm<0>();  // b's loads, the only ones in flight
        }
        lds_barrier();
        if (!AHEAD && b + 1 < nb) issue(b + 1, smem + ((b + 1) & 1) * GM_WA, tails + next * GM_TB);
        gemm_mfma<NMT>(smem + (b & 1) * GM_WA, wave, lane, dc, hc);
        if constexpr (decltype(fold)::value) {
            gemm_fold<NMT>(tails + prev * GM_TB, lane, dp, hp, acc);
        }
        if constexpr (AHEAD) {
            lds_barrier();
            if (b + 2 < nb) issue(b + 2, smem + (b & 1) * GM_WA, tails + prev * GM_TB);
        }
        slot = next;
    };
    step(std::false_type{}, 0, d0, h0, d1, h1);
    for (int b = 1; b < nb; b += 2) {
        step(std::true_type{}, b, d1, h1, d0, h0);
        if (b + 1 < nb) step(std::true_type{}, b + 1, d0, h0, d1, h1);
    }
    if constexpr (!AHEAD) lds_barrier();
    const int last = slot == 0 ? 2 : slot - 1;  // the slot of nb - 1
    if (nb & 1)
        gemm_fold<NMT>(tails + last * GM_TB, lane, d0, h0, acc);
    else
        gemm_fold<NMT>(tails + last * GM_TB, lane, d1, h1, acc);
}

__global__ __launch_bounds__(64 * GM_WAVES) void k_gemm_q4k(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: slot choices in SGPRs
    const int n0 = blockIdx.x * GM_ROWS, t0 = blockIdx.y * GM_TT;
    const int T = active_rows(g.active, 0, g.T);
    if (t0 >= T) return;  // uniform: a token tile past the step's active rows
    const GemmSlots sl = gemm_slots(g, wave, lane, n0, t0);
    const int live = sl.nw + GM_ASLOT / GM_WAVES + sl.nt;  // loads per stage of this wavefront
    v4f acc[GM_MT][GM_NT];
#pragma unroll
    for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) acc[mt][nt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    auto issue = [&](int b, uint8_t* stage, uint8_t* tail) { gemm_issue(g, sl, wave, lane, b, t0, stage, tail); };
    // the 16-token tiles holding active rows (a last tile of fewer rows computes only those)
    switch ((T - t0 < GM_TT ? T - t0 + 15 : GM_TT) / 16) {
        case 1: gemm_loop<1, true>(g.nb, live, smem, wave, lane, issue, acc); break;
        case 2: gemm_loop<2, true>(g.nb, live, smem, wave, lane, issue, acc); break;
        case 3: gemm_loop<3, true>(g.nb, live, smem, wave, lane, issue, acc); break;
        default: gemm_loop<GM_MT, true>(g.nb, live, smem, wave, lane, issue, acc); break;
    }

    const int c = lane & 15, p = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) {
            const int n = n0 + 16 * GM_NT * wave + 16 * nt + c;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + 16 * mt + 4 * p + i;
                if (t < T && n < g.N) g.y[(int64_t)t * g.N + n] = acc[mt][nt][i];
            }
        }
}

bool gemm_q4k_supported(int n_out, int k) {
    return k >= 256 && k % 256 == 0 && n_out > 0 &&
           (uint64_t)n_out * (uint64_t)(k / 256) * 144u < (1ull << 32);
}

void launch_gemm_q4k(int layout, const uint8_t* W, int n_out, int k, GemmAct a, int T, float* y,
                     hipStream_t stream, const uint32_t* active) {
    GemmArgs g{};
    g.active = active;
    g.W = W;
    g.layout = layout;
    g.codes = a.codes;
    g.tail = a.tail;
    g.y = y;
    g.N = n_out;
    g.T = T;
    g.nb = k / 256;
    g.tpad = a.tpad;
    g.rb = (uint32_t)(k / 256) * 144u;
    // once per process, thread-safe (a function-local static); a refusal shows as the launch's error
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)k_gemm_q4k, hipFuncAttributeMaxDynamicSharedMemorySize, GM_LOOP_LDS);
    (void)attr;
    const dim3 grid((unsigned)((n_out + GM_ROWS - 1) / GM_ROWS), (unsigned)(a.tpad / GM_TT));
    hipLaunchKernelGGL(k_gemm_q4k, grid, dim3(64 * GM_WAVES), GM_LOOP_LDS, stream, g);
}

// ============================================================================================
// The MoE layer at many tokens: the grouped expert FFN on the same matrix cores
// ============================================================================================
//
// Each expert's entries (the packed lists of k_moe_pack: offsets, slots) are padded to whole
// 64-entry tiles: tile i belongs to expert tile_e[i], and its padded position p = 64 i + t holds
// entry offsets[e] + p - pad_off[e] when that is below offsets[e + 1] (padding positions'
// outputs are dropped).  An entry's row is quantized exactly as the expert quantizes it
// (moe.rs:479-492), which depends on the row alone, so:
//   gate/up: the tokens' rows are quantized to Q8_K once, in the GEMM layout, and each stage
//     gathers position p's row from its entry's token (slots[i] / top_k); a workgroup takes
//     (tile, 128 weight rows); its 256-row weight tile is those 128 rows of the tile's gate
//     matrix followed by the same 128 rows of its up matrix, so wavefronts 0-3 hold g and
//     wavefronts 4-7 hold u of the same outputs, and h = silu(g) * u per entry
//     (moe.rs:529-551);
//   down: the entries' h rows quantized at their padded positions; (tile, 256 rows) of the
//     expert's down matrix; each output goes to its entry's slot (moe.rs:500-515).
// Every product is the Gemv value (the same exact sums and term fold as the dense GEMM).

// One workgroup: an inclusive scan of the experts' tile counts (E <= 256).
__global__ __launch_bounds__(256) void k_moe_tiles(const uint32_t* __restrict__ offsets, int n_experts,
                                                   const uint32_t* __restrict__ err, MoeTiles mt) {
    __shared__ uint32_t cnt[256];
    const int e = threadIdx.x;
    const bool bad = err[0] != 0;  // uniform: the layer writes nothing
    const uint32_t n = (!bad && e < n_experts) ? offsets[e + 1] - offsets[e] : 0u;
    const uint32_t tiles = (n + 63u) / 64u;
    cnt[e] = tiles;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t v = e >= off ? cnt[e - off] : 0u;
        __syncthreads();
        cnt[e] += v;
        __syncthreads();
    }
    const uint32_t end = cnt[e], begin = end - tiles;
    if (e < n_experts) mt.pad_off[e] = 64u * begin;
    if (e == n_experts - 1) {
        mt.pad_off[n_experts] = 64u * end;
        mt.n_tiles[0] = end;
    }
    for (uint32_t i = begin; i < end; ++i) mt.tile_e[i] = (uint32_t)e;
}

void launch_moe_tiles(const uint32_t* offsets, int n_experts, const uint32_t* err, MoeTiles mt,
                      hipStream_t stream) {
    hipLaunchKernelGGL(k_moe_tiles, dim3(1), dim3(256), 0, stream, offsets, n_experts, err, mt);
}

// The entries' h rows at their padded positions (row i of h for entry i).  Positions in tiles
// past the used ones are not written (no workgroup reads them).
template <int BPW>
__global__ __launch_bounds__(256) void k_moe_gemm_act(const float* __restrict__ h, int k,
                                                      const uint32_t* __restrict__ offsets, MoeTiles mt,
                                                      const uint32_t* __restrict__ err, GemmAct a) {
    if (err[0]) return;
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t ng = (k / 256 + BPW - 1) / BPW;
    if (item >= ng * a.tpad) return;
    const uint32_t tile = (uint32_t)(item - (item / a.tpad) * a.tpad) / 64u;
    if (tile >= mt.n_tiles[0]) return;  // a tile past the used ones: nothing reads it
    gemm_act_blocks<BPW>(k / 256, item, a, lane, [&](int pos) {
        const uint32_t e = mt.tile_e[tile];
        const uint32_t i = offsets[e] + ((uint32_t)pos - mt.pad_off[e]);
        return i < offsets[e + 1] ? h + (int64_t)i * k : nullptr;
    });
}

void launch_moe_gemm_act(const float* h, int k, const uint32_t* offsets, MoeTiles mt, const uint32_t* err,
                         GemmAct a, hipStream_t stream) {
    const int64_t items = gemm_act_items(k / 256, a.tpad);
    if (items == 0) return;
    const dim3 grid((unsigned)((items + 3) / 4));
    if (gemm_act_bpw(k / 256, a.tpad) == 4)
        hipLaunchKernelGGL(k_moe_gemm_act<4>, grid, dim3(256), 0, stream, h, k, offsets, mt, err, a);
    else
        hipLaunchKernelGGL(k_moe_gemm_act<1>, grid, dim3(256), 0, stream, h, k, offsets, mt, err, a);
}

struct MoeGemmArgs {
    const uint8_t* W0;  // gate (MODE 0) or down (MODE 1), stacked by expert
    const uint8_t* W1;  // up (MODE 0)
    uint64_t ebytes;    // bytes of one expert's matrix
    GemmAct act;
    int nb;             // super-blocks along k
    uint32_t rb;        // weight row bytes
    int row_tiles;      // workgroups per entry tile
    const uint32_t* offsets;
    MoeTiles mt;
    const uint32_t* err;
    const uint32_t* slots;
    float* out;         // h [entries][cols] (MODE 0) or out [slots][cols] (MODE 1)
    int cols;           // inter (MODE 0) or hidden (MODE 1)
    int layout;         // LAYOUT_SOURCE or LAYOUT_TILE64 (the row tiles are whole 64-row runs)
    int top_k;          // MODE 0: act holds the tokens' rows, position p of a tile reads its
                        // entry's token slots[i] / top_k
};

// MODE 0 (gate/up, 128 weight rows of each per workgroup) or 1 (down, 256 rows).
template <int MODE>
__global__ __launch_bounds__(64 * GM_WAVES) void k_moe_gemm(MoeGemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    if (g.err[0]) return;
    const int tile = (int)blockIdx.x / g.row_tiles, rt = (int)blockIdx.x - tile * g.row_tiles;
    if ((uint32_t)tile >= g.mt.n_tiles[0]) return;  // uniform per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t e = g.mt.tile_e[tile];
    const int t0 = 64 * tile;
    const uint32_t i0 = g.offsets[e] + ((uint32_t)t0 - g.mt.pad_off[e]);
    const uint32_t left = g.offsets[e + 1] - i0;
    const int nvalid = left < 64u ? (int)left : 64;
    constexpr int ROWS = MODE == 0 ? GM_ROWS / 2 : GM_ROWS;  // rows of each matrix
    const uint8_t* b0 = g.W0 + (uint64_t)e * g.ebytes + (uint64_t)rt * ROWS * g.rb;
    const uint8_t* b1 = MODE == 0 ? g.W1 + (uint64_t)e * g.ebytes + (uint64_t)rt * ROWS * g.rb : b0;
    // the weight tile's 256 rows: MODE 0 rows 0-127 of b0 then rows 0-127 of b1 (slots
    // 0..GM_WSLOT/2-1 hold exactly the first 128 rows: 128 * 9 chunks = 18 slots of 64)
    GemmArgs ga{};
    ga.layout = g.layout;
    ga.N = GM_ROWS;
    ga.rb = g.rb;
    ga.codes = g.act.codes;
    ga.tail = g.act.tail;
    ga.tpad = g.act.tpad;
    ga.nb = g.nb;
    GemmSlots sl = gemm_slots(ga, wave, lane, 0, t0);
    static_assert(GM_ROWS / 2 * 9 % 64 == 0, "gate and up halves on whole slots");
    constexpr int HALF_SLOTS = GM_ROWS / 2 * 9 / 64;
    bool upper[GM_WPW];
#pragma unroll
    for (int u = 0; u < GM_WPW; ++u) {
        upper[u] = MODE == 0 && wave + GM_WAVES * u >= HALF_SLOTS;
        if (upper[u]) sl.woff[u] -= (uint32_t)(GM_ROWS / 2) * g.rb;
    }
    // MODE 0 gathers each position's token row from the tokens' quantized rows: code slot u of
    // this lane is 16-byte chunk q of position pa, which holds chunk q ^ (pa & 15) (the stage's
    // bank skew) and sits in the token's row at chunk (q ^ (pa & 15)) ^ (tok & 15) (the row's
    // own skew); tail: wavefronts 0-1 the s2 halves, 2 the scales, 3 the code sums, one position
    // a lane (padding positions read token 0; their outputs are dropped)
    const uint32_t tp = (uint32_t)g.act.tpad;
    auto token_of = [&](int pa) -> uint32_t {
        return pa < nvalid ? g.slots[i0 + (uint32_t)pa] / (uint32_t)g.top_k : 0u;
    };
    uint32_t aoff[GM_ASLOT / GM_WAVES];
    uint32_t toff = 0;
    if constexpr (MODE == 0) {
#pragma unroll
        for (int u = 0; u < GM_ASLOT / GM_WAVES; ++u) {
            const int pa = 2 * (wave + GM_WAVES * u) + (lane >> 5), q = lane & 31;
            const uint32_t tok = token_of(pa);
            aoff[u] = tok * 512u + 16u * (uint32_t)((q ^ (pa & 15)) ^ (int)(tok & 15u));
        }
        if (wave < 2) {
            toff = token_of((64 * wave + lane) >> 1) * 32u + 16u * (uint32_t)(lane & 1);
        } else if (wave < 4) {
            toff = tp * (wave == 2 ? 32u : 36u) + token_of(lane) * 4u;
        }
    }
    // super-block b of the tile's rows: 144 b on in GGUF order, 64 rows' blocks on in TILE64
    const size_t bstep = g.layout == LAYOUT_TILE64 ? (size_t)TILE64_ROWS * 144 : 144;
    auto issue = [&](int b, uint8_t* stage, uint8_t* tail) {
        const uint8_t* w0 = b0 + bstep * (size_t)b;
        const uint8_t* w1 = b1 + bstep * (size_t)b;
        const uint32_t st = lds_addr(stage);
#pragma unroll
        for (int u = 0; u < GM_WPW; ++u)
            if (u < sl.nw) lds_dma16(sl.woff[u], upper[u] ? w1 : w0, st + 1024u * (uint32_t)(wave + GM_WAVES * u));
        if constexpr (MODE == 0) {
            // super-block bases in 64 bits (2 * hidden * tp bytes of codes may pass 2^32);
            // the offsets within one super-block's rows stay below 2^25
            const uint8_t* ab = g.act.codes + (size_t)b * tp * 512u;
            const uint8_t* tb = g.act.tail + (size_t)b * tp * (uint32_t)GM_TAIL_ROW;
#pragma unroll
            for (int u = 0; u < GM_ASLOT / GM_WAVES; ++u) {
                const int gs = wave + GM_WAVES * u;
                lds_dma16(aoff[u], ab, st + (uint32_t)GM_WB + 1024u * (uint32_t)gs);
            }
            const uint32_t tl = lds_addr(tail);
            if (wave < 2)
                lds_dma16(toff, tb, tl + 1024u * (uint32_t)wave);
            else if (wave < 4)
                lds_dma4(toff, tb, tl + (wave == 2 ? 2048u : 2304u));
        } else {
            const uint8_t* ab = g.act.codes + ((size_t)b * g.act.tpad + t0) * 512;
            const uint8_t* tb = g.act.tail + (size_t)b * g.act.tpad * GM_TAIL_ROW;
#pragma unroll
            for (int u = 0; u < GM_ASLOT / GM_WAVES; ++u) {
                const int gs = wave + GM_WAVES * u;
                lds_dma16(16u * (uint32_t)lane, ab + 1024 * gs, st + (uint32_t)GM_WB + 1024u * (uint32_t)gs);
            }
            if (sl.ton) lds_dma16(sl.toff, tb, lds_addr(tail) + 1024u * (uint32_t)wave);
        }
    };
    v4f acc[GM_MT][GM_NT];
#pragma unroll
    for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < GM_NT; ++nt) acc[mt][nt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // the 16-token tiles holding entries (the padding of an expert's last tile is not computed;
    // its outputs are dropped)
    switch ((nvalid + 15) / 16) {
        case 1: gemm_loop<1, false>(g.nb, 0, smem, wave, lane, issue, acc); break;
        case 2: gemm_loop<2, false>(g.nb, 0, smem, wave, lane, issue, acc); break;
        case 3: gemm_loop<3, false>(g.nb, 0, smem, wave, lane, issue, acc); break;
        default: gemm_loop<GM_MT, false>(g.nb, 0, smem, wave, lane, issue, acc); break;
    }
    const int c = lane & 15, p = lane >> 4;
    if constexpr (MODE == 0) {
        // u (wavefronts 4-7) through LDS to the wavefronts holding g of the same outputs
        float* ux = reinterpret_cast<float*>(smem);  // [64 tokens][128 rows]
        if (wave >= GM_WAVES / 2) {
#pragma unroll
            for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < GM_NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        ux[(16 * mt + 4 * p + i) * ROWS + 16 * GM_NT * (wave - GM_WAVES / 2) + 16 * nt + c] = acc[mt][nt][i];
        }
        lds_barrier();
        if (wave < GM_WAVES / 2) {
#pragma unroll
            for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < GM_NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = 16 * mt + 4 * p + i, r = 16 * GM_NT * wave + 16 * nt + c;
                        if (t < nvalid) {
                            const float u = ux[t * ROWS + r];
                            g.out[(int64_t)(i0 + t) * g.cols + rt * ROWS + r] = ref_silu(acc[mt][nt][i]) * u;
                        }
                    }
        }
    } else {
#pragma unroll
        for (int mt = 0; mt < GM_MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < GM_NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * mt + 4 * p + i, r = 16 * GM_NT * wave + 16 * nt + c;
                    if (t < nvalid) g.out[(int64_t)g.slots[i0 + t] * g.cols + rt * ROWS + r] = acc[mt][nt][i];
                }
    }
}

void launch_moe_gemm(int mode, const uint8_t* w0, const uint8_t* w1, int n_experts, int rows, int k,
                     GemmAct act, int max_tiles, const uint32_t* offsets, MoeTiles mt, const uint32_t* err,
                     const uint32_t* slots, float* out, hipStream_t stream, int top_k, int layout) {
    static_assert(GM_ROWS % (2 * TILE64_ROWS) == 0, "row tiles of whole TILE64 runs");
    MoeGemmArgs g;
    g.top_k = top_k;
    g.layout = layout == LAYOUT_TILE64 ? (int)LAYOUT_TILE64 : (int)LAYOUT_SOURCE;
    g.W0 = w0;
    g.W1 = w1;
    g.nb = k / 256;
    g.rb = (uint32_t)g.nb * 144u;
    g.ebytes = (uint64_t)rows * g.rb;
    g.act = act;
    g.row_tiles = mode == 0 ? rows / (GM_ROWS / 2) : rows / GM_ROWS;
    g.offsets = offsets;
    g.mt = mt;
    g.err = err;
    g.slots = slots;
    g.out = out;
    g.cols = rows;
    const dim3 grid((unsigned)(max_tiles * g.row_tiles));
    if (mode == 0) {
        static const hipError_t ok0 = hipFuncSetAttribute((const void*)k_moe_gemm<0>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, GM_LOOP_LDS);
        (void)ok0;  // a refusal shows as the launch's error
        hipLaunchKernelGGL(k_moe_gemm<0>, grid, dim3(64 * GM_WAVES), GM_LOOP_LDS, stream, g);
    } else {
        static const hipError_t ok1 = hipFuncSetAttribute((const void*)k_moe_gemm<1>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, GM_LOOP_LDS);
        (void)ok1;
        hipLaunchKernelGGL(k_moe_gemm<1>, grid, dim3(64 * GM_WAVES), GM_LOOP_LDS, stream, g);
    }
}

// Row tiles: gate/up 128 rows, down 256.
bool moe_gemm_supported(int hidden, int inter) { return hidden % GM_ROWS == 0 && inter % (GM_ROWS / 2) == 0; }

}  // namespace syn
