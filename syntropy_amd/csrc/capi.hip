// The C ABI (include/syntropy_hip.h): argument checks, then the kernel launchers.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/syntropy_hip.h"
#include "capi_rows.hpp"
#include "kernels.hpp"

#define SYN_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SYN_E_DEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
    return SYN_OK;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// The weight view of a matrix of need_w bytes (nblocks blocks) in `layout`.  A SOURCE view may run
// past the matrix.  The repacks are shape-free and place bytes by the total length they were
// given (SPLIT's scale section starts after every block's codes; X8's final run of fewer than 8
// super-blocks has its own stride), so a repacked view must be the repack of this matrix alone:
// exactly need_w bytes for SPLIT, and for X8 when the block count is not a multiple of 8.
int check_view(const char* W, uint32_t layout, uint64_t w_bytes, uint64_t need_w, uint64_t nblocks) {
    if (w_bytes < need_w)
        return fail(SYN_E_INVALID, "%s: the weight view holds %llu bytes, the matrix %llu", W,
                    (unsigned long long)w_bytes, (unsigned long long)need_w);
    const bool exact = layout == SYN_LAYOUT_SPLIT || (layout == SYN_LAYOUT_X8 && nblocks % 8 != 0);
    if (exact && w_bytes != need_w)
        return fail(SYN_E_INVALID,
                    "%s: a layout-%u weight view must be the repack of the matrix alone: %llu bytes, not %llu", W,
                    layout, (unsigned long long)need_w, (unsigned long long)w_bytes);
    return SYN_OK;
}

bool gemv_type(int32_t t) { return t == SYN_Q4_0 || t == SYN_Q8_0 || t == SYN_Q4_K; }
bool float_type(int32_t t) { return t == SYN_F16 || t == SYN_BF16; }

int check_gemv_shape(const char* what, int32_t wtype, uint32_t rows, uint32_t k_in) {
    if (!gemv_type(wtype) && !float_type(wtype))
        return fail(SYN_E_UNSUPPORTED, "%s: weight type %d is not F16, BF16, Q4_0, Q8_0 or Q4_K", what, wtype);
    const int be = syn::block_elems(wtype);
    if (k_in % (uint32_t)be)
        return fail(SYN_E_INVALID, "%s: a row of %u weights is not whole %d-weight blocks", what, k_in, be);
    if ((uint64_t)rows * k_in > (1ull << 40)) return fail(SYN_E_INVALID, "%s: rows * k_in too large", what);
    return SYN_OK;
}

// Q4_K calls of at least this many activation rows run on the matrix cores (k_gemm_q4k); the
// value of every output is the same either way.
constexpr uint32_t GEMM_MIN_ROWS = 32;

uint64_t gemm_tpad(uint32_t rows) { return ((uint64_t)rows + 63) / 64 * 64; }

bool use_gemm(int32_t wtype, uint32_t rows, uint32_t n_out, uint32_t k_in) {
    return wtype == SYN_Q4_K && rows >= GEMM_MIN_ROWS && syn::gemm_q4k_supported((int)n_out, (int)k_in) &&
           gemm_tpad(rows) * (k_in / 256) < (1ull << 31);
}

// Q4_K Gemv calls of 2 to 31 rows run on the decode expert kernel (the matrix as one expert,
// the rows as its entries: the int8 matrix cores over four-row groups).
bool q4k_dense(int32_t wtype, uint32_t rows, uint32_t k_in) {
    return wtype == SYN_Q4_K && rows >= 2 && rows < GEMM_MIN_ROWS && k_in > 0 && k_in % 256 == 0;
}

// Workspace of a Gemv call: the larger of the two activation layouts when the call may take
// the matrix-core path (the bytes do not depend on n_out, which the workspace query lacks).
uint64_t gemv_ws_bytes(int32_t wtype, uint32_t rows, uint32_t k_in) {
    uint64_t b = syn::act_layout(syn::act_kind(wtype), rows, k_in).bytes;
    if (q4k_dense(wtype, rows, k_in)) {
        const uint64_t m = syn::moe_act_bytes(rows, (int)k_in);
        if (m > b) b = m;
    }
    if (use_gemm(wtype, rows, 1, k_in)) {
        const uint64_t g = syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in);
        if (g > b) b = g;
    }
    return b;
}

int check_gemm_shape(const char* what, uint32_t rows, uint32_t k_in) {
    if (k_in == 0 || k_in % 256) return fail(SYN_E_INVALID, "%s: k_in %u is not whole 256-weight super-blocks", what, k_in);
    if (gemm_tpad(rows) * (k_in / 256) >= (1ull << 31)) return fail(SYN_E_INVALID, "%s: rows * k_in too large", what);
    return SYN_OK;
}

}  // namespace

SYN_EXPORT const char* syn_last_error(void) { return g_last_error.c_str(); }
SYN_EXPORT int syn_version(void) { return 100; }

SYN_EXPORT int syn_gemv_workspace_bytes(int32_t wtype, uint32_t rows, uint32_t k_in,
                                        uint64_t* bytes) {
    if (int rc = check_gemv_shape("syn_gemv_workspace_bytes", wtype, rows, k_in)) return rc;
    if (!bytes) return fail(SYN_E_INVALID, "syn_gemv_workspace_bytes: null output");
    *bytes = gemv_ws_bytes(wtype, rows, k_in);
    return SYN_OK;
}

SYN_EXPORT int syn_act_quantize(int32_t wtype, const float* x, uint32_t rows, uint32_t k_in,
                                void* ws, uint64_t ws_bytes, void* stream) {
    const char* W = "syn_act_quantize";
    if (int rc = check_gemv_shape(W, wtype, rows, k_in)) return rc;
    if (float_type(wtype)) return fail(SYN_E_UNSUPPORTED, "%s: F16 and BF16 products take F32 activations", W);
    const uint64_t need = syn::act_layout(syn::act_kind(wtype), rows, k_in).bytes;
    if ((uint64_t)rows * k_in == 0) return SYN_OK;
    if (!x || !ws) return fail(SYN_E_INVALID, "%s: null x or workspace", W);
    if (!aligned(x, 16) || !aligned(ws, 256))
        return fail(SYN_E_INVALID, "%s: x must be 16-byte and the workspace 256-byte aligned", W);
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    syn::launch_act_quant(syn::act_kind(wtype), x, rows, k_in, (uint8_t*)ws, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_gemv_quantized(int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                                  uint32_t k_in, const void* ws, uint64_t ws_bytes, uint32_t rows,
                                  float* y, void* stream) {
    const char* W = "syn_gemv_quantized";
    if (int rc = check_gemv_shape(W, wtype, rows, k_in)) return rc;
    if (float_type(wtype)) return fail(SYN_E_UNSUPPORTED, "%s: F16 and BF16 products take F32 activations", W);
    if (rows == 0 || n_out == 0) return SYN_OK;
    if (n_out > (1u << 30)) return fail(SYN_E_INVALID, "%s: n_out too large", W);
    const uint64_t row_bytes = (uint64_t)k_in / syn::block_elems(wtype) * syn::block_bytes(wtype);
    const uint64_t need_w = row_bytes * n_out;
    const uint64_t need_ws = syn::act_layout(syn::act_kind(wtype), rows, k_in).bytes;
    if (!y || (need_w && !w) || (need_ws && !ws)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (w_bytes < need_w)
        return fail(SYN_E_INVALID, "%s: the weight view holds %llu bytes, the matrix %llu", W,
                    (unsigned long long)w_bytes, (unsigned long long)need_w);
    if (ws_bytes < need_ws)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need_ws);
    if (!aligned(ws, 256) || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: the workspace must be 256-byte and y 4-byte aligned", W);
    if (wtype == SYN_Q4_K && rows == 1 && k_in > 0 && syn::q4k_dec_supported((int)k_in) && aligned(w, 16))
        syn::launch_gemv_q4k_dec_ws((const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws, y,
                                    (hipStream_t)stream);
    else
        syn::launch_gemv_q(wtype, (const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws,
                           (int)rows, y, (hipStream_t)stream);
    return check_launch(W);
}

namespace {
// Q4_K rows 2..31: the rows to Q8_K in the expert kernels' layout, then the dense expert product
// (layout 0: GGUF order; 1: X8).  Operands already checked by the caller.
int q4k_dense_rows(const char* W, int x8, const void* w, uint32_t n_out, uint32_t k_in, const float* x,
                   uint32_t rows, float* y, void* ws, void* stream, const uint32_t* active) {
    if (x8 && syn::gemv_q4k_x8_rows_pick((int)n_out, (int)k_in, (int)rows)) {  // the one-row kernel's loads
        if (syn::gemv_q4k_x8_rows_fused((int)k_in, (int)rows)) {  // one launch: the rows quantized in its workgroups
            syn::launch_gemv_q4k_x8_rows((const uint8_t*)w, (int)n_out, (int)k_in, nullptr, x, (int)rows, y,
                                         (hipStream_t)stream, active);
            return check_launch(W);
        }
        syn::launch_act_quant(syn::ACT_Q8K, x, rows, k_in, (uint8_t*)ws, (hipStream_t)stream);
        if (int rc = check_launch(W)) return rc;
        syn::launch_gemv_q4k_x8_rows((const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws, nullptr, (int)rows,
                                     y, (hipStream_t)stream, active);
        return check_launch(W);
    }
    const syn::MoeAct a = syn::moe_act_at((uint8_t*)ws, rows, (int)k_in);
    syn::launch_moe_gather_q8k(x, nullptr, (int)rows, 1, (int)k_in, nullptr, a, 0, (hipStream_t)stream, nullptr);
    if (int rc = check_launch(W)) return rc;
    syn::launch_q4k_dense_rows((const uint8_t*)w, x8, (int)n_out, (int)k_in, a, (int)rows, y, (hipStream_t)stream,
                               active);
    return check_launch(W);
}
}  // namespace

int syn_gemv_rows(int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                        uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws,
                        uint64_t ws_bytes, void* stream, const uint32_t* active) {
    const char* W = "syn_gemv";
    if (int rc = check_gemv_shape(W, wtype, rows, k_in)) return rc;
    if (rows == 0 || n_out == 0) return SYN_OK;
    const uint64_t row_bytes = (uint64_t)k_in / syn::block_elems(wtype) * syn::block_bytes(wtype);
    const bool gemm = use_gemm(wtype, rows, n_out, k_in) && aligned(w, 16);
    uint64_t need_ws = gemm ? syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in)
                            : syn::act_layout(syn::act_kind(wtype), rows, k_in).bytes;
    if (!gemm && q4k_dense(wtype, rows, k_in) && syn::moe_act_bytes(rows, (int)k_in) > need_ws)
        need_ws = syn::moe_act_bytes(rows, (int)k_in);
    if (!y || (row_bytes * n_out && !w)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (w_bytes < row_bytes * n_out)
        return fail(SYN_E_INVALID, "%s: the weight view holds %llu bytes, the matrix %llu", W,
                    (unsigned long long)w_bytes, (unsigned long long)(row_bytes * n_out));
    if (ws_bytes < need_ws)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need_ws);
    if (k_in && (!x || (!ws && !float_type(wtype)))) return fail(SYN_E_INVALID, "%s: null x or workspace", W);
    if (float_type(wtype)) {
        // F32 activations straight into the FMA accumulators: no workspace
        if ((k_in && (!x || !aligned(x, 4) || !aligned(w, 2))) || !aligned(y, 4))
            return fail(SYN_E_INVALID, "%s: x and y must be 4-byte and w 2-byte aligned", W);
        syn::launch_gemv_float(wtype, (const uint8_t*)w, (int)n_out, (int)k_in, x, (int)rows, y, (hipStream_t)stream,
                                active);
        return check_launch(W);
    }
    if ((k_in && (!aligned(x, 16) || !aligned(ws, 256))) || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: x must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
    if (wtype == SYN_Q4_K && rows == 1 && k_in > 0 && syn::q4k_dec_supported((int)k_in) && aligned(w, 16)) {
        // one launch: the workgroups quantize the row into LDS themselves
        syn::launch_gemv_q4k_dec_f32((const uint8_t*)w, (int)n_out, (int)k_in, x, y, (hipStream_t)stream, active);
        return check_launch(W);
    }
    if (gemm) {
        const syn::GemmAct a = syn::gemm_act_at((uint8_t*)ws, (int64_t)gemm_tpad(rows), (int)k_in);
        syn::launch_gemm_act(x, (int)rows, (int)k_in, a, (hipStream_t)stream, active);
        if (int rc = check_launch(W)) return rc;
        syn::launch_gemm_q4k(SYN_LAYOUT_SOURCE, (const uint8_t*)w, (int)n_out, (int)k_in, a, (int)rows, y,
                             (hipStream_t)stream, active);
        return check_launch(W);
    }
    if (q4k_dense(wtype, rows, k_in) && aligned(w, 16) && row_bytes * n_out < (1ull << 32))
        return q4k_dense_rows(W, 0, w, n_out, k_in, x, rows, y, ws, stream, active);
    if (k_in) {
        syn::launch_act_quant(syn::act_kind(wtype), x, rows, k_in, (uint8_t*)ws, (hipStream_t)stream);
        if (int rc = check_launch(W)) return rc;
    }
    syn::launch_gemv_q(wtype, (const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws, (int)rows,
                       y, (hipStream_t)stream, active);
    return check_launch(W);
}

SYN_EXPORT int syn_gemv(int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                        uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws,
                        uint64_t ws_bytes, void* stream) {
    return syn_gemv_rows(wtype, w, w_bytes, n_out, k_in, x, rows, y, ws, ws_bytes, stream, nullptr);
}

SYN_EXPORT int syn_gemm_workspace_bytes(uint32_t rows, uint32_t k_in, uint64_t* bytes) {
    const char* W = "syn_gemm_workspace_bytes";
    if (int rc = check_gemm_shape(W, rows, k_in)) return rc;
    if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
    *bytes = syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in);
    return SYN_OK;
}

SYN_EXPORT int syn_gemm_act_quantize(const float* x, uint32_t rows, uint32_t k_in, void* ws,
                                     uint64_t ws_bytes, void* stream) {
    const char* W = "syn_gemm_act_quantize";
    if (int rc = check_gemm_shape(W, rows, k_in)) return rc;
    if (rows == 0) return SYN_OK;
    const uint64_t need = syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in);
    if (!x || !ws) return fail(SYN_E_INVALID, "%s: null x or workspace", W);
    if (!aligned(x, 16) || !aligned(ws, 256))
        return fail(SYN_E_INVALID, "%s: x must be 16-byte and the workspace 256-byte aligned", W);
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    syn::launch_gemm_act(x, (int)rows, (int)k_in,
                         syn::gemm_act_at((uint8_t*)ws, (int64_t)gemm_tpad(rows), (int)k_in), (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_gemm_q4k_quantized(const void* w, uint64_t w_bytes, uint32_t n_out, uint32_t k_in,
                                      const void* ws, uint64_t ws_bytes, uint32_t rows, float* y,
                                      void* stream) {
    const char* W = "syn_gemm_q4k_quantized";
    if (int rc = check_gemm_shape(W, rows, k_in)) return rc;
    if (rows == 0 || n_out == 0) return SYN_OK;
    if (!syn::gemm_q4k_supported((int)n_out, (int)k_in))
        return fail(SYN_E_UNSUPPORTED, "%s: a %u x %u matrix is larger than 4 GiB", W, n_out, k_in);
    const uint64_t need_w = (uint64_t)n_out * (k_in / 256) * 144;
    const uint64_t need = syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in);
    if (!w || !ws || !y) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (w_bytes < need_w)
        return fail(SYN_E_INVALID, "%s: the weight view holds %llu bytes, the matrix %llu", W,
                    (unsigned long long)w_bytes, (unsigned long long)need_w);
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!aligned(w, 16) || !aligned(ws, 256) || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: w must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
    syn::launch_gemm_q4k(SYN_LAYOUT_SOURCE, (const uint8_t*)w, (int)n_out, (int)k_in,
                         syn::gemm_act_at((uint8_t*)ws, (int64_t)gemm_tpad(rows), (int)k_in), (int)rows, y,
                         (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_gemv_batch_workspace_bytes(uint32_t n, const uint32_t* k_in, uint64_t* bytes) {
    const char* W = "syn_gemv_batch_workspace_bytes";
    if (n > SYN_BATCH) return fail(SYN_E_UNSUPPORTED, "%s: at most %d problems", W, SYN_BATCH);
    if (!bytes || (n && !k_in)) return fail(SYN_E_INVALID, "%s: null argument", W);
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (k_in[i] % 256) return fail(SYN_E_INVALID, "%s: k_in[%u] = %u is not whole 256-weight blocks", W, i, k_in[i]);
        total += syn::act_layout(syn::ACT_Q8K, 1, k_in[i]).bytes;
    }
    *bytes = total;
    return SYN_OK;
}

namespace {

// Shared checks of the grouped entry points: problem i's quantized row sits at ws + off[i].
int batch_setup(const char* W, uint32_t layout, uint32_t n, const int32_t* wtypes, const void* const* w,
                const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in, void* ws,
                uint64_t ws_bytes, uint64_t* off) {
    if (n > SYN_BATCH) return fail(SYN_E_UNSUPPORTED, "%s: at most %d problems", W, SYN_BATCH);
    if (!k_in || (w && (!wtypes || !w_bytes || !n_out))) return fail(SYN_E_INVALID, "%s: null argument array", W);
    uint64_t need = 0;
    if (int rc = syn_gemv_batch_workspace_bytes(n, k_in, &need)) return rc;
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!ws || !aligned(ws, 256)) return fail(SYN_E_INVALID, "%s: the workspace must be 256-byte aligned", W);
    uint64_t o = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (k_in[i] == 0 || k_in[i] > 16384) return fail(SYN_E_UNSUPPORTED, "%s: k_in[%u] = %u (1..16384)", W, i, k_in[i]);
        if (w) {
            if (wtypes[i] != SYN_Q4_K) return fail(SYN_E_UNSUPPORTED, "%s: problem %u is not Q4_K", W, i);
            if (n_out[i] == 0 || n_out[i] > (1u << 28)) return fail(SYN_E_INVALID, "%s: n_out[%u] = %u", W, i, n_out[i]);
            const uint64_t need_w = (uint64_t)k_in[i] / 256 * 144 * n_out[i];
            if (int rc = check_view(W, layout, w_bytes[i], need_w, need_w / 144)) return rc;
            if (!w[i] || !aligned(w[i], 16)) return fail(SYN_E_INVALID, "%s: problem %u: W must be a 16-byte aligned pointer", W, i);
        }
        off[i] = o;
        o += syn::act_layout(syn::ACT_Q8K, 1, k_in[i]).bytes;
    }
    return SYN_OK;
}

int batch_quantize(const char* W, uint32_t n, const uint32_t* k_in, const float* const* x,
                   uint8_t* ws, const uint64_t* off, hipStream_t st) {
    const float* xp[SYN_BATCH];
    uint8_t* wsm[SYN_BATCH];
    int kk[SYN_BATCH];
    for (uint32_t i = 0; i < n; ++i) {
        if (!x[i] || !aligned(x[i], 16)) return fail(SYN_E_INVALID, "%s: x[%u] must be a 16-byte aligned pointer", W, i);
        xp[i] = x[i];
        wsm[i] = ws + off[i];
        kk[i] = (int)k_in[i];
    }
    syn::launch_act_quant_batch((int)n, xp, kk, wsm, st);
    return check_launch(W);
}

int batch_gemv(const char* W, int layout, uint32_t n, const void* const* w, const uint32_t* n_out,
               const uint32_t* k_in, const uint8_t* ws, const uint64_t* off, float* const* y,
               hipStream_t st) {
    if (layout != SYN_LAYOUT_SOURCE && layout != SYN_LAYOUT_X8)
        return fail(SYN_E_UNSUPPORTED, "%s: weight layout %d", W, layout);
    const uint8_t* wp[SYN_BATCH];
    const uint8_t* wsp[SYN_BATCH];
    float* yp[SYN_BATCH];
    int no[SYN_BATCH], kk[SYN_BATCH];
    for (uint32_t i = 0; i < n; ++i) {
        if (!y[i] || !aligned(y[i], 4)) return fail(SYN_E_INVALID, "%s: y[%u] must be a 4-byte aligned pointer", W, i);
        wp[i] = (const uint8_t*)w[i];
        wsp[i] = ws + off[i];
        yp[i] = y[i];
        no[i] = (int)n_out[i];
        kk[i] = (int)k_in[i];
    }
    syn::launch_gemv_q4k_batch(layout, (int)n, wp, no, kk, wsp, yp, st);
    return check_launch(W);
}

}  // namespace

SYN_EXPORT int syn_act_quantize_batch(uint32_t n, const uint32_t* k_in, const float* const* x,
                                      void* ws, uint64_t ws_bytes, void* stream) {
    const char* W = "syn_act_quantize_batch";
    if (n == 0) return SYN_OK;
    if (!x) return fail(SYN_E_INVALID, "%s: null argument array", W);
    uint64_t off[SYN_BATCH];
    if (int rc = batch_setup(W, SYN_LAYOUT_SOURCE, n, nullptr, nullptr, nullptr, nullptr, k_in, ws, ws_bytes, off)) return rc;
    return batch_quantize(W, n, k_in, x, (uint8_t*)ws, off, (hipStream_t)stream);
}

SYN_EXPORT int syn_gemv_batch_quantized_layout(uint32_t layout, uint32_t n, const int32_t* wtypes,
                                               const void* const* w, const uint64_t* w_bytes,
                                               const uint32_t* n_out, const uint32_t* k_in, const void* ws,
                                               uint64_t ws_bytes, float* const* y, void* stream) {
    const char* W = "syn_gemv_batch_quantized";
    if (n == 0) return SYN_OK;
    if (!w || !y) return fail(SYN_E_INVALID, "%s: null argument array", W);
    uint64_t off[SYN_BATCH];
    if (int rc = batch_setup(W, layout, n, wtypes, w, w_bytes, n_out, k_in, (void*)ws, ws_bytes, off)) return rc;
    return batch_gemv(W, (int)layout, n, w, n_out, k_in, (const uint8_t*)ws, off, y, (hipStream_t)stream);
}

SYN_EXPORT int syn_gemv_batch_quantized(uint32_t n, const int32_t* wtypes, const void* const* w,
                                        const uint64_t* w_bytes, const uint32_t* n_out,
                                        const uint32_t* k_in, const void* ws, uint64_t ws_bytes,
                                        float* const* y, void* stream) {
    return syn_gemv_batch_quantized_layout(SYN_LAYOUT_SOURCE, n, wtypes, w, w_bytes, n_out, k_in, ws, ws_bytes,
                                           y, stream);
}

namespace {

// The grouped Gemv on F32 rows.  fuse = 0: one batched Q8_K quantization into the workspace,
// then the grouped GEMV (the faster pair for a whole layer); fuse = 1: one launch whose
// workgroups quantize their problem's row into LDS themselves (one launch fewer, for a lone
// Gemv); the workspace is still sized and checked.
int gemv_batch_f32(const char* W, uint32_t layout, uint32_t n, const int32_t* wtypes, const void* const* w,
                   const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in, const float* const* x,
                   float* const* y, void* ws, uint64_t ws_bytes, void* stream, bool fuse,
                   const uint32_t* active = nullptr) {
    if (n == 0) return SYN_OK;
    if (!w || !x || !y) return fail(SYN_E_INVALID, "%s: null argument array", W);
    if (layout != SYN_LAYOUT_SOURCE && layout != SYN_LAYOUT_X8)
        return fail(SYN_E_UNSUPPORTED, "%s: weight layout %u", W, layout);
    uint64_t off[SYN_BATCH];
    if (int rc = batch_setup(W, layout, n, wtypes, w, w_bytes, n_out, k_in, ws, ws_bytes, off)) return rc;
    if (!fuse || layout != SYN_LAYOUT_X8) {
        if (int rc = batch_quantize(W, n, k_in, x, (uint8_t*)ws, off, (hipStream_t)stream)) return rc;
        return batch_gemv(W, (int)layout, n, w, n_out, k_in, (const uint8_t*)ws, off, y, (hipStream_t)stream);
    }
    const uint8_t* wp[SYN_BATCH];
    const float* xp[SYN_BATCH];
    float* yp[SYN_BATCH];
    int no[SYN_BATCH], kk[SYN_BATCH];
    for (uint32_t i = 0; i < n; ++i) {
        if (!x[i] || !aligned(x[i], 16)) return fail(SYN_E_INVALID, "%s: x[%u] must be a 16-byte aligned pointer", W, i);
        if (!y[i] || !aligned(y[i], 4)) return fail(SYN_E_INVALID, "%s: y[%u] must be a 4-byte aligned pointer", W, i);
        if (!syn::gemv_q4k_batch_fusable((int)k_in[i])) return fail(SYN_E_UNSUPPORTED, "%s: k_in[%u] = %u", W, i, k_in[i]);
        wp[i] = (const uint8_t*)w[i];
        xp[i] = x[i];
        yp[i] = y[i];
        no[i] = (int)n_out[i];
        kk[i] = (int)k_in[i];
    }
    syn::launch_gemv_q4k_batch_f32(wp, (int)n, no, kk, xp, yp, (hipStream_t)stream, active);
    return check_launch(W);
}

}  // namespace

SYN_EXPORT int syn_gemv_batch_layout(uint32_t layout, uint32_t n, const int32_t* wtypes, const void* const* w,
                                     const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                                     const float* const* x, float* const* y, void* ws, uint64_t ws_bytes,
                                     void* stream) {
    return gemv_batch_f32("syn_gemv_batch", layout, n, wtypes, w, w_bytes, n_out, k_in, x, y, ws, ws_bytes, stream,
                          false);
}

SYN_EXPORT int syn_gemv_batch(uint32_t n, const int32_t* wtypes, const void* const* w,
                              const uint64_t* w_bytes, const uint32_t* n_out, const uint32_t* k_in,
                              const float* const* x, float* const* y, void* ws, uint64_t ws_bytes,
                              void* stream) {
    return syn_gemv_batch_layout(SYN_LAYOUT_SOURCE, n, wtypes, w, w_bytes, n_out, k_in, x, y, ws, ws_bytes,
                                 stream);
}

// ---- weight layouts -----------------------------------------------------------------------------

namespace {
int check_repack(const char* W, uint32_t layout, const void* src, void* dst, uint64_t bytes) {
    if (layout != SYN_LAYOUT_X8) return fail(SYN_E_UNSUPPORTED, "%s: layout %u (1: X8)", W, layout);
    if (bytes % 144) return fail(SYN_E_INVALID, "%s: %llu bytes are not whole Q4_K super-blocks", W, (unsigned long long)bytes);
    if (bytes && (!src || !dst)) return fail(SYN_E_INVALID, "%s: null buffer", W);
    if (bytes && src == dst) return fail(SYN_E_INVALID, "%s: the repack is not in place", W);
    return SYN_OK;
}
}  // namespace

SYN_EXPORT int syn_q4k_repack(uint32_t layout, const void* src, void* dst, uint64_t bytes, int32_t inverse,
                              void* stream) {
    const char* W = "syn_q4k_repack";
    if (int rc = check_repack(W, layout, src, dst, bytes)) return rc;
    if (!aligned(src, 16) || !aligned(dst, 16)) return fail(SYN_E_INVALID, "%s: buffers must be 16-byte aligned", W);
    syn::launch_q4k_x8((const uint8_t*)src, (uint8_t*)dst, bytes / 144, inverse != 0, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_q4k_repack_host(uint32_t layout, const void* src, void* dst, uint64_t bytes, int32_t inverse) {
    const char* W = "syn_q4k_repack_host";
    if (int rc = check_repack(W, layout, src, dst, bytes)) return rc;
    const uint64_t nblocks = bytes / 144;
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* d = (uint8_t*)dst;
    for (uint64_t g = 0; g < nblocks; ++g)
        for (int q = 0; q < 9; ++q) {
            const uint64_t to = syn::x8_chunk_offset(g, q, nblocks), from = g * 144 + 16 * (uint64_t)q;
            memcpy(d + (inverse ? from : to), s + (inverse ? to : from), 16);
        }
    return SYN_OK;
}

namespace {
int check_tile64(const char* W, const void* src, void* dst, uint64_t bytes, uint32_t k_in) {
    if (k_in == 0 || k_in % 256 || k_in > 65536)
        return fail(SYN_E_INVALID, "%s: k_in %u must be whole super-blocks, at most 65536", W, k_in);
    const uint64_t run = (uint64_t)syn::TILE64_ROWS * (k_in / 256) * 144;
    if (bytes % run)
        return fail(SYN_E_INVALID, "%s: %llu bytes are not whole runs of 64 rows of %u values", W,
                    (unsigned long long)bytes, k_in);
    if (bytes && (!src || !dst)) return fail(SYN_E_INVALID, "%s: null buffer", W);
    if (bytes && src == dst) return fail(SYN_E_INVALID, "%s: the repack is not in place", W);
    return SYN_OK;
}
}  // namespace

SYN_EXPORT int syn_q4k_tile64_repack(const void* src, void* dst, uint64_t bytes, uint32_t k_in, int32_t inverse,
                                     void* stream) {
    const char* W = "syn_q4k_tile64_repack";
    if (int rc = check_tile64(W, src, dst, bytes, k_in)) return rc;
    if (!aligned(src, 16) || !aligned(dst, 16)) return fail(SYN_E_INVALID, "%s: buffers must be 16-byte aligned", W);
    syn::launch_tile64_repack((const uint8_t*)src, (uint8_t*)dst, bytes, (int)k_in, inverse != 0, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_q4k_tile64_repack_host(const void* src, void* dst, uint64_t bytes, uint32_t k_in, int32_t inverse) {
    const char* W = "syn_q4k_tile64_repack_host";
    if (int rc = check_tile64(W, src, dst, bytes, k_in)) return rc;
    const uint64_t rb = (uint64_t)(k_in / 256) * 144, rows = bytes / rb;
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* d = (uint8_t*)dst;
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t b = 0; b < k_in / 256; ++b) {
            const uint64_t g = r * rb + 144 * b, t = syn::tile64_row_offset(r, rb) + (uint64_t)syn::TILE64_ROWS * 144 * b;
            memcpy(d + (inverse ? g : t), s + (inverse ? t : g), 144);
        }
    return SYN_OK;
}

namespace {
int check_split_repack(const char* W, uint32_t layout, int32_t wtype, const void* src, void* dst, uint64_t bytes) {
    if (layout != SYN_LAYOUT_SPLIT) return fail(SYN_E_UNSUPPORTED, "%s: layout %u (2: SPLIT)", W, layout);
    if (wtype != SYN_Q8_0 && wtype != SYN_Q4_0)
        return fail(SYN_E_UNSUPPORTED, "%s: weight type %d (the SPLIT layout holds Q8_0 or Q4_0)", W, wtype);
    const uint64_t bb = (uint64_t)syn::split_code_bytes(wtype) + 2;
    if (bytes % bb)
        return fail(SYN_E_INVALID, "%s: %llu bytes are not whole %llu-byte blocks", W, (unsigned long long)bytes,
                    (unsigned long long)bb);
    if (bytes && (!src || !dst)) return fail(SYN_E_INVALID, "%s: null buffer", W);
    if (bytes && src == dst) return fail(SYN_E_INVALID, "%s: the repack is not in place", W);
    return SYN_OK;
}
}  // namespace

SYN_EXPORT int syn_split_repack(uint32_t layout, int32_t wtype, const void* src, void* dst, uint64_t bytes,
                                int32_t inverse, void* stream) {
    const char* W = "syn_split_repack";
    if (int rc = check_split_repack(W, layout, wtype, src, dst, bytes)) return rc;
    syn::launch_split_repack(wtype, (const uint8_t*)src, (uint8_t*)dst, bytes, inverse != 0, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_split_repack_host(uint32_t layout, int32_t wtype, const void* src, void* dst, uint64_t bytes,
                                     int32_t inverse) {
    const char* W = "syn_split_repack_host";
    if (int rc = check_split_repack(W, layout, wtype, src, dst, bytes)) return rc;
    const uint64_t cb = (uint64_t)syn::split_code_bytes(wtype), nblocks = bytes / (cb + 2);
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* d = (uint8_t*)dst;
    for (uint64_t g = 0; g < nblocks; ++g) {
        const uint64_t gguf = g * (cb + 2), codes = g * cb, scale = cb * nblocks + 2 * g;
        if (!inverse) {
            memcpy(d + codes, s + gguf + 2, cb);
            memcpy(d + scale, s + gguf, 2);
        } else {
            memcpy(d + gguf + 2, s + codes, cb);
            memcpy(d + gguf, s + scale, 2);
        }
    }
    return SYN_OK;
}

// Gemv over weights in a repacked layout.  Q4_K in X8: one row runs the grouped decode kernel,
// 2 to 31 rows the decode expert kernel (int8 matrix cores), more rows the matrix-core GEMM (which
// needs rows of whole 8-block runs: k_in a multiple of 2048).  Q8_0 / Q4_0 in SPLIT: Q8_0 activation
// rows, the split decode kernel for up to 8 rows at a time, the int8 matrix-core GEMM where its
// LDS-staged form takes the shape (rows of whole 4-block stages) and is the faster, and for other
// Q8_0 shapes from 9 rows.
constexpr uint32_t SPLIT_GEMM_MIN_ROWS = 9;
constexpr uint32_t SPLIT_GEMM_MAX_ROWS = 65535u * 32u;  // the GEMM grid's token tiles

namespace {
// Whether the staged GEMM beats the split decode kernel at 2 to 16 rows (one 16-token tile), from
// estimated microseconds fitted on MI355X timings of both kernels with the weights read from
// HBM (Q8_0 and Q4_0, 4096 to 14336 rows of 4096 to 14336 values).  Split decode kernel, per launch of r <= 8 rows over M million
// weights: a + read M + per M r (Q4_0: 2.4, 0.089, 0.038; Q8_0: 3.2, 0.141, 0.034, or 0.070
// per row and million weights when the activation rows do not fit in LDS and are read from
// global memory).  The GEMM's estimate is gemm_q8_cost_us (gemv_split.hip): flat in the rows up
// to 16 and following the row length, while the decode kernel's grows with the rows; beyond 16
// rows the GEMM is always the faster.  All produce the same bits.
bool staged_faster(int32_t wtype, uint32_t n_out, uint32_t k_in, uint32_t rows) {
    if (rows > 16) return true;
    const bool q8 = wtype == SYN_Q8_0;
    const double M = (double)n_out * (double)k_in * 1e-6;
    double gemv = 0.0;
    for (uint32_t r0 = 0; r0 < rows; r0 += 8) {
        const uint32_t r = rows - r0 < 8 ? rows - r0 : 8;
        const double per = !q8 ? 0.038 : syn::gemv_split_staged((int)wtype, (int)r, (int)k_in) ? 0.034 : 0.070;
        gemv += (q8 ? 3.2 : 2.4) + (q8 ? 0.141 : 0.089) * M + per * M * (double)r;
    }
    return syn::gemm_q8_cost_us((int)wtype, (int)n_out, (int)k_in, (int)rows) < gemv;
}

// Rows on the int8 matrix cores: where the LDS-staged GEMM takes the shape and is the faster
// (above), else Q8_0 from 9 rows on the register-staged GEMM.
bool split_gemm(int32_t wtype, uint32_t n_out, uint32_t k_in, uint32_t rows) {
    if (wtype != SYN_Q8_0 && wtype != SYN_Q4_0) return false;
    if (rows >= 2 && syn::gemm_q8_staged_fits((int)wtype, (int)n_out, (int)k_in, (int)rows))
        return staged_faster(wtype, n_out, k_in, rows);
    return wtype == SYN_Q8_0 && rows >= SPLIT_GEMM_MIN_ROWS;
}

// The products over a SPLIT matrix from rows already quantized to Q8_0 blocks in ws.
void split_products(int32_t wtype, const void* w, uint32_t n_out, uint32_t k_in, const void* ws, uint32_t rows,
                    float* y, void* stream, const uint32_t* active) {
    if (split_gemm(wtype, n_out, k_in, rows))
        syn::launch_gemm_q8_split((int)wtype, (const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws, (int)rows,
                                  y, (hipStream_t)stream, active);
    else
        syn::launch_gemv_split(wtype, (const uint8_t*)w, (int)n_out, (int)k_in, (const uint8_t*)ws, (int)rows, y,
                               (hipStream_t)stream, active);
}
}  // namespace
SYN_EXPORT int syn_gemv_layout_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t k_in,
                                               uint64_t* bytes) {
    const char* W = "syn_gemv_layout_workspace_bytes";
    if (layout == SYN_LAYOUT_SOURCE) return syn_gemv_workspace_bytes(wtype, rows, k_in, bytes);
    if (layout == SYN_LAYOUT_SPLIT && (wtype == SYN_Q8_0 || wtype == SYN_Q4_0)) {
        if (int rc = check_gemv_shape(W, wtype, rows, k_in)) return rc;
        if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
        if (k_in / 32 > (1u << 24)) return fail(SYN_E_UNSUPPORTED, "%s: k_in %u too large", W, k_in);
        *bytes = syn::act_layout(syn::ACT_Q8_0, rows, k_in).bytes;
        return SYN_OK;
    }
    if (layout != SYN_LAYOUT_X8 || wtype != SYN_Q4_K)
        return fail(SYN_E_UNSUPPORTED, "%s: layout %u of weight type %d", W, layout, wtype);
    if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
    if (rows <= 1) {
        if (k_in == 0 || k_in % 256 || k_in > 16384) return fail(SYN_E_UNSUPPORTED, "%s: k_in %u (256..16384, whole super-blocks)", W, k_in);
        *bytes = syn::act_layout(syn::ACT_Q8K, 1, k_in).bytes;
        return SYN_OK;
    }
    if (q4k_dense(wtype, rows, k_in)) {  // 2..31 rows: the decode expert kernel
        *bytes = syn::moe_act_bytes(rows, (int)k_in);
        return SYN_OK;
    }
    if (k_in % 2048) return fail(SYN_E_UNSUPPORTED, "%s: the layout-1 GEMM takes k_in in multiples of 2048, not %u", W, k_in);
    if (int rc = check_gemm_shape(W, rows, k_in)) return rc;
    *bytes = syn::gemm_act_bytes((int64_t)gemm_tpad(rows), (int)k_in);
    return SYN_OK;
}

int syn_gemv_layout_rows(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                               uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                               void* stream, const uint32_t* active) {
    const char* W = "syn_gemv_layout";
    if (layout == SYN_LAYOUT_SOURCE)
        return syn_gemv_rows(wtype, w, w_bytes, n_out, k_in, x, rows, y, ws, ws_bytes, stream, active);
    uint64_t need = 0;
    if (int rc = syn_gemv_layout_workspace_bytes(layout, wtype, rows, k_in, &need)) return rc;
    if (rows == 0 || n_out == 0) return SYN_OK;
    if (layout == SYN_LAYOUT_SPLIT) {
        const uint64_t need_w = (uint64_t)n_out * (k_in / 32) * (syn::split_code_bytes(wtype) + 2);
        if (!w || !y || (k_in && (!x || !ws))) return fail(SYN_E_INVALID, "%s: null operand", W);
        if (int rc = check_view(W, layout, w_bytes, need_w, (uint64_t)n_out * (k_in / 32))) return rc;
        if (ws_bytes < need)
            return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                        (unsigned long long)ws_bytes, (unsigned long long)need);
        if (!aligned(w, 16) || (k_in && (!aligned(x, 16) || !aligned(ws, 256))) || !aligned(y, 4))
            return fail(SYN_E_INVALID, "%s: w and x must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
        if ((uint64_t)n_out * rows > (1ull << 40)) return fail(SYN_E_INVALID, "%s: rows * n_out too large", W);
        if (split_gemm(wtype, n_out, k_in, rows) && rows > SPLIT_GEMM_MAX_ROWS)
            return fail(SYN_E_UNSUPPORTED, "%s: %u rows (the GEMM takes %u)", W, rows, SPLIT_GEMM_MAX_ROWS);
        if (rows == 1 && k_in && !split_gemm(wtype, n_out, k_in, rows) && syn::gemv_split_fused_fits((int)wtype, (int)k_in)) {
            // one row: quantized inside the product's workgroups, one launch
            syn::launch_gemv_split_fused((int)wtype, (const uint8_t*)w, (int)n_out, (int)k_in, x, y, (hipStream_t)stream,
                                         active);
            return check_launch(W);
        }
        if (k_in) {
            syn::launch_act_quant(syn::ACT_Q8_0, x, rows, k_in, (uint8_t*)ws, (hipStream_t)stream);
            if (int rc = check_launch(W)) return rc;
        }
        split_products(wtype, w, n_out, k_in, ws, rows, y, stream, active);
        return check_launch(W);
    }
    if (rows == 1) {
        const float* xs[1] = {x};
        float* ys[1] = {y};
        const void* ws_[1] = {w};
        const int32_t ts[1] = {wtype};
        const uint64_t wb[1] = {w_bytes};
        return gemv_batch_f32(W, layout, 1, ts, ws_, wb, &n_out, &k_in, xs, ys, ws, ws_bytes, stream, true, active);
    }
    if (q4k_dense(wtype, rows, k_in)) {
        const uint64_t need_w = (uint64_t)n_out * (k_in / 256) * 144;
        if (!w || !x || !ws || !y) return fail(SYN_E_INVALID, "%s: null operand", W);
        if (int rc = check_view(W, layout, w_bytes, need_w, need_w / 144)) return rc;
        if (ws_bytes < need)
            return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                        (unsigned long long)ws_bytes, (unsigned long long)need);
        if (!aligned(w, 16) || !aligned(x, 16) || !aligned(ws, 256) || !aligned(y, 4))
            return fail(SYN_E_INVALID, "%s: w and x must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
        return q4k_dense_rows(W, 1, w, n_out, k_in, x, rows, y, ws, stream, active);
    }
    if (!syn::gemm_q4k_supported((int)n_out, (int)k_in))
        return fail(SYN_E_UNSUPPORTED, "%s: a %u x %u matrix is larger than 4 GiB", W, n_out, k_in);
    const uint64_t need_w = (uint64_t)n_out * (k_in / 256) * 144;
    if (!w || !x || !ws || !y) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (int rc = check_view(W, layout, w_bytes, need_w, need_w / 144)) return rc;
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!aligned(w, 16) || !aligned(x, 16) || !aligned(ws, 256) || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: w and x must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
    const syn::GemmAct a = syn::gemm_act_at((uint8_t*)ws, (int64_t)gemm_tpad(rows), (int)k_in);
    syn::launch_gemm_act(x, (int)rows, (int)k_in, a, (hipStream_t)stream, active);
    if (int rc = check_launch(W)) return rc;
    syn::launch_gemm_q4k(SYN_LAYOUT_X8, (const uint8_t*)w, (int)n_out, (int)k_in, a, (int)rows, y, (hipStream_t)stream,
                         active);
    return check_launch(W);
}

SYN_EXPORT int syn_gemv_layout(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                               uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                               void* stream) {
    return syn_gemv_layout_rows(layout, wtype, w, w_bytes, n_out, k_in, x, rows, y, ws, ws_bytes, stream, nullptr);
}

// The product alone, over rows syn_act_quantize already quantized (Q8_0 blocks for the SPLIT
// layout's Q8_0 and Q4_0 matrices).
SYN_EXPORT int syn_gemv_quantized_layout(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes,
                                         uint32_t n_out, uint32_t k_in, const void* ws, uint64_t ws_bytes,
                                         uint32_t rows, float* y, void* stream) {
    const char* W = "syn_gemv_quantized_layout";
    if (layout == SYN_LAYOUT_SOURCE)
        return syn_gemv_quantized(wtype, w, w_bytes, n_out, k_in, ws, ws_bytes, rows, y, stream);
    if (layout != SYN_LAYOUT_SPLIT)
        return fail(SYN_E_UNSUPPORTED, "%s: layout %u (0: SOURCE, 2: SPLIT)", W, layout);
    uint64_t need = 0;
    if (int rc = syn_gemv_layout_workspace_bytes(layout, wtype, rows, k_in, &need)) return rc;
    if (rows == 0 || n_out == 0) return SYN_OK;
    const uint64_t need_w = (uint64_t)n_out * (k_in / 32) * (syn::split_code_bytes(wtype) + 2);
    if (!w || !y || (k_in && !ws)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (int rc = check_view(W, layout, w_bytes, need_w, (uint64_t)n_out * (k_in / 32))) return rc;
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!aligned(w, 16) || (k_in && !aligned(ws, 256)) || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: w must be 16-byte, the workspace 256-byte and y 4-byte aligned", W);
    if ((uint64_t)n_out * rows > (1ull << 40)) return fail(SYN_E_INVALID, "%s: rows * n_out too large", W);
    if (split_gemm(wtype, n_out, k_in, rows) && rows > SPLIT_GEMM_MAX_ROWS)
        return fail(SYN_E_UNSUPPORTED, "%s: %u rows (the GEMM takes %u)", W, rows, SPLIT_GEMM_MAX_ROWS);
    split_products(wtype, w, n_out, k_in, ws, rows, y, stream, nullptr);
    return check_launch(W);
}

// ---- syn_gemv_layout without a caller workspace ---------------------------------------------
// The workspace lives in `scratch`, one array per device that holds it until the process ends.
// Host code never passes the array's name to a kernel (that is a host-side stand-in, not a
// device address): the device address comes from hipGetSymbolAddress, once per device, with
// that device current, and every use goes through it.
namespace {

constexpr uint64_t SCRATCH_BYTES = 8ull << 20;
constexpr int SCRATCH_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

std::atomic<void*> g_scratch[SCRATCH_DEVICES];
std::mutex g_scratch_init;

// The current device's scratch address; null with the message set on failure.
void* scratch_of_current_device(const char* W) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_DEVICES) {
        fail(SYN_E_DEVICE, "%s: no current device below %d", W, SCRATCH_DEVICES);
        return nullptr;
    }
    if (void* p = g_scratch[dev].load(std::memory_order_acquire)) return p;
    std::lock_guard<std::mutex> lock(g_scratch_init);
    if (void* p = g_scratch[dev].load(std::memory_order_acquire)) return p;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        fail(SYN_E_DEVICE, "%s: hipGetSymbolAddress(scratch) on device %d: %s", W, dev, hipGetErrorString(e));
        return nullptr;
    }
    g_scratch[dev].store(p, std::memory_order_release);
    return p;
}

}  // namespace

SYN_EXPORT uint64_t syn_gemv_layout_noalloc_max_workspace(void) { return SCRATCH_BYTES; }

SYN_EXPORT int syn_gemv_layout_noalloc(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes,
                                       uint32_t n_out, uint32_t k_in, const float* x, uint32_t rows, float* y,
                                       void* stream) {
    const char* W = "syn_gemv_layout_noalloc";
    uint64_t need = 0;
    if (int rc = syn_gemv_layout_workspace_bytes(layout, wtype, rows, k_in, &need)) return rc;
    if (need > SCRATCH_BYTES)
        return fail(SYN_E_UNSUPPORTED, "%s: %u rows of %u need a %llu-byte workspace; the device scratch holds %llu",
                    W, rows, k_in, (unsigned long long)need, (unsigned long long)SCRATCH_BYTES);
    if (rows == 0 || n_out == 0) return SYN_OK;
    void* ws = scratch_of_current_device(W);
    if (!ws) return SYN_E_DEVICE;
    // every byte the kernels read from the workspace is written earlier in the same call
    return syn_gemv_layout_rows(layout, wtype, w, w_bytes, n_out, k_in, x, rows, y, ws, SCRATCH_BYTES, stream,
                                nullptr);
}

SYN_EXPORT int syn_gate_up_act_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t n_out,
                                               uint32_t k_in, uint64_t* bytes) {
    const char* W = "syn_gate_up_act_workspace_bytes";
    if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
    uint64_t g = 0;
    if (int rc = syn_gemv_layout_workspace_bytes(layout, wtype, rows, k_in, &g)) return rc;
    // the Gemv's workspace, then the stacked product [rows][2 n_out]
    *bytes = syn::align_up(g, 256) + 8ull * rows * n_out;
    return SYN_OK;
}

int syn_gate_up_act_rows(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                               uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                               void* stream, const uint32_t* active) {
    const char* W = "syn_gate_up_act";
    uint64_t need = 0;
    if (int rc = syn_gate_up_act_workspace_bytes(layout, wtype, rows, n_out, k_in, &need)) return rc;
    if (rows == 0 || n_out == 0) return SYN_OK;
    if (n_out > (1u << 29)) return fail(SYN_E_INVALID, "%s: n_out too large", W);
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!ws || !aligned(ws, 256) || !y || !aligned(y, 4))
        return fail(SYN_E_INVALID, "%s: the workspace must be 256-byte and y 4-byte aligned", W);
    if (layout == SYN_LAYOUT_X8 && wtype == SYN_Q4_K && rows == 1 && syn::gemv_q4k_batch_fusable((int)k_in)) {
        // one launch: the row quantized in every workgroup, gate and up rows side by side, silu(g) u
        const uint64_t need_w = 2ull * n_out * (k_in / 256) * 144;
        if (!w || !x) return fail(SYN_E_INVALID, "%s: null operand", W);
        if (int rc = check_view(W, layout, w_bytes, need_w, need_w / 144)) return rc;
        if (!aligned(w, 16) || !aligned(x, 16)) return fail(SYN_E_INVALID, "%s: w and x must be 16-byte aligned", W);
        syn::launch_gate_up_q4k_f32((const uint8_t*)w, (int)n_out, (int)k_in, x, y, (hipStream_t)stream, active);
        return check_launch(W);
    }
    uint64_t g = 0;
    (void)syn_gemv_layout_workspace_bytes(layout, wtype, rows, k_in, &g);
    float* y2 = (float*)((uint8_t*)ws + syn::align_up(g, 256));
    if (int rc = syn_gemv_layout_rows(layout, wtype, w, w_bytes, 2 * n_out, k_in, x, rows, y2, ws, g, stream, active))
        return rc;
    syn::launch_silu_mul(y2, (int)rows, (int)n_out, y, (hipStream_t)stream, active);
    return check_launch(W);
}

SYN_EXPORT int syn_gate_up_act(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                               uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                               void* stream) {
    return syn_gate_up_act_rows(layout, wtype, w, w_bytes, n_out, k_in, x, rows, y, ws, ws_bytes, stream, nullptr);
}

// ---- measurement ----------------------------------------------------------------------------

SYN_EXPORT uint64_t syn_hbm_read_probe_sink_words(uint64_t bytes) { return syn::hbm_read_probe_workgroups(bytes); }

SYN_EXPORT int syn_hbm_read_probe(const void* src, uint64_t bytes, uint32_t* sink, void* stream) {
    const char* W = "syn_hbm_read_probe";
    if (bytes % 16) return fail(SYN_E_INVALID, "%s: %llu bytes are not whole 16-byte chunks", W, (unsigned long long)bytes);
    if (bytes && (!src || !sink)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(SYN_E_INVALID, "%s: src must be 16-byte aligned", W);
    syn::launch_hbm_read_probe((const uint8_t*)src, bytes, sink, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_div_forms_check(unsigned long long* counts, void* stream) {
    const char* W = "syn_div_forms_check";
    if (!counts || !aligned(counts, 8)) return fail(SYN_E_INVALID, "%s: counts must be 8-byte aligned device memory", W);
    syn::launch_div_forms_check(counts, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT uint64_t syn_hbm_read_runs_sink_words(uint64_t bytes) { return syn::hbm_read_runs_units(bytes); }

SYN_EXPORT int syn_hbm_read_runs(uint32_t waves, const void* src, uint64_t bytes, uint32_t* sink, void* stream) {
    const char* W = "syn_hbm_read_runs";
    if (waves != 1 && waves != 8) return fail(SYN_E_UNSUPPORTED, "%s: %u wavefronts a workgroup (1 or 8)", W, waves);
    if (bytes % 16) return fail(SYN_E_INVALID, "%s: %llu bytes are not whole 16-byte chunks", W, (unsigned long long)bytes);
    if (bytes && (!src || !sink)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(SYN_E_INVALID, "%s: src must be 16-byte aligned", W);
    syn::launch_hbm_read_runs((int)waves, (const uint8_t*)src, bytes, sink, (hipStream_t)stream);
    return check_launch(W);
}

// ---- RmsNorm and Logits ------------------------------------------------------------------

SYN_EXPORT int syn_rms_norm(const float* x, const float* g, uint32_t rows, uint32_t n, float eps, float* y,
                            void* stream) {
    const char* W = "syn_rms_norm";
    if (n > (uint32_t)syn::NORM_MAX_COLS) return fail(SYN_E_UNSUPPORTED, "%s: rows of %u values (at most %d)", W, n, syn::NORM_MAX_COLS);
    if (rows == 0 || n == 0) return SYN_OK;
    if (!x || !g || !y) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(x, 4) || !aligned(g, 4) || !aligned(y, 4)) return fail(SYN_E_INVALID, "%s: operands must be 4-byte aligned", W);
    syn::launch_rms_norm(x, g, (int)rows, (int)n, eps, y, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_logits_workspace_bytes(uint32_t layout, int32_t wtype, uint32_t rows, uint32_t vocab,
                                          uint32_t hidden, uint64_t* bytes) {
    const char* W = "syn_logits_workspace_bytes";
    if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
    (void)vocab;
    uint64_t g = 0;
    if (int rc = syn_gemv_layout_workspace_bytes(layout, wtype, rows, hidden, &g)) return rc;
    // the normalised rows [rows][hidden] F32, then the head product's workspace
    *bytes = syn::align_up(4ull * rows * hidden, 256) + g;
    return SYN_OK;
}

int syn_logits_rows(uint32_t layout, int32_t wtype, const void* head, uint64_t head_bytes, uint32_t vocab,
                    uint32_t hidden, const float* g, float eps, const float* x, uint32_t rows, float* y, void* ws,
                    uint64_t ws_bytes, void* stream, const uint32_t* active) {
    const char* W = "syn_logits";
    uint64_t need = 0;
    if (int rc = syn_logits_workspace_bytes(layout, wtype, rows, vocab, hidden, &need)) return rc;
    if (hidden > (uint32_t)syn::NORM_MAX_COLS)
        return fail(SYN_E_UNSUPPORTED, "%s: hidden %u (at most %d)", W, hidden, syn::NORM_MAX_COLS);
    if (rows == 0 || vocab == 0) return SYN_OK;
    if (!x || !g || !ws) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (ws_bytes < need)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)need);
    if (!aligned(ws, 256) || !aligned(x, 4) || !aligned(g, 4))
        return fail(SYN_E_INVALID, "%s: the workspace must be 256-byte, x and g 4-byte aligned", W);
    float* h = (float*)ws;
    const uint64_t hb = syn::align_up(4ull * rows * hidden, 256);
    syn::launch_rms_norm(x, g, (int)rows, (int)hidden, eps, h, (hipStream_t)stream, active);
    if (int rc = check_launch(W)) return rc;
    return syn_gemv_layout_rows(layout, wtype, head, head_bytes, vocab, hidden, h, rows, y, (uint8_t*)ws + hb,
                                ws_bytes - hb, stream, active);
}

SYN_EXPORT int syn_logits(uint32_t layout, int32_t wtype, const void* head, uint64_t head_bytes, uint32_t vocab,
                          uint32_t hidden, const float* g, float eps, const float* x, uint32_t rows, float* y,
                          void* ws, uint64_t ws_bytes, void* stream) {
    return syn_logits_rows(layout, wtype, head, head_bytes, vocab, hidden, g, eps, x, rows, y, ws, ws_bytes, stream,
                           nullptr);
}

SYN_EXPORT int syn_quantize(int32_t wtype, const float* x, uint64_t n, void* out,
                            uint64_t out_bytes, void* stream) {
    const char* W = "syn_quantize";
    if (!gemv_type(wtype)) return fail(SYN_E_UNSUPPORTED, "%s: weight type %d", W, wtype);
    const int be = syn::block_elems(wtype);
    if (n % (uint64_t)be) return fail(SYN_E_INVALID, "%s: %llu values are not whole %d-value blocks", W, (unsigned long long)n, be);
    const uint64_t need = n / be * syn::block_bytes(wtype);
    if (out_bytes < need) return fail(SYN_E_INVALID, "%s: output holds %llu bytes, needs %llu", W, (unsigned long long)out_bytes, (unsigned long long)need);
    if (n == 0) return SYN_OK;
    if (!x || !out) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(x, 4) || !aligned(out, 2)) return fail(SYN_E_INVALID, "%s: misaligned operand", W);
    syn::launch_quantize(wtype, x, n, (uint8_t*)out, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_dequantize(int32_t wtype, const void* src, uint64_t src_bytes, float* out,
                              void* stream) {
    const char* W = "syn_dequantize";
    if (!gemv_type(wtype)) return fail(SYN_E_UNSUPPORTED, "%s: weight type %d", W, wtype);
    const int bb = syn::block_bytes(wtype);
    if (src_bytes % (uint64_t)bb) return fail(SYN_E_INVALID, "%s: %llu bytes are not whole %d-byte blocks", W, (unsigned long long)src_bytes, bb);
    if (src_bytes == 0) return SYN_OK;
    if (!src || !out) return fail(SYN_E_INVALID, "%s: null operand", W);
    syn::launch_dequantize(wtype, (const uint8_t*)src, src_bytes / bb * syn::block_elems(wtype), out,
                           (hipStream_t)stream);
    return check_launch(W);
}

// ============================================================================================
// MoE
// ============================================================================================

namespace {

// The expert FFN runs on the prefill GEMM (entries padded to 64-entry tiles per expert) once the
// experts average this many entries; below it, on the grouped decode kernels.
constexpr uint64_t MOE_GEMM_MIN_AVG = 32;

bool moe_use_gemm(uint32_t n_experts, uint32_t top_k, uint32_t hidden, uint32_t inter, uint32_t rows) {
    return (uint64_t)rows * top_k >= MOE_GEMM_MIN_AVG * n_experts && syn::moe_gemm_supported((int)hidden, (int)inter);
}

// Workspace of syn_moe_grouped: offsets, slots, the error word, then
//   decode kernels: the packed entries' Q8_K activations, the entries' h rows and their Q8_K;
//   GEMM path: the tile table (padded offsets, tile experts, tile count), the entries' rows in
//   the GEMM layout at their padded positions, h, and h in the GEMM layout;
// every section on 256 bytes.
struct MoeWs {
    uint64_t offsets, slots, err, xq, h, hq, bytes;
    bool gemm;
    uint64_t pad_off, tile_e, n_tiles;
    int max_tiles;
};
MoeWs moe_ws(uint32_t n_experts, uint32_t top_k, uint32_t hidden, uint32_t inter, uint32_t rows) {
    MoeWs m{};
    const uint64_t ent = (uint64_t)rows * top_k;
    uint64_t o = 0;
    m.offsets = o;
    o = syn::align_up(o + 4ull * (n_experts + 1), 256);
    m.slots = o;
    o = syn::align_up(o + 4ull * ent, 256);
    m.err = o;  // error word, then the largest expert's entry count
    o = syn::align_up(o + 8, 256);
    m.gemm = moe_use_gemm(n_experts, top_k, hidden, inter, rows);
    if (m.gemm) {
        m.max_tiles = (int)((ent + 63) / 64 + n_experts);
        const int64_t tpad = 64ll * m.max_tiles;
        m.pad_off = o;
        o = syn::align_up(o + 4ull * (n_experts + 1), 256);
        m.tile_e = o;
        o = syn::align_up(o + 4ull * m.max_tiles, 256);
        m.n_tiles = o;
        o = syn::align_up(o + 4, 256);
        m.xq = o;
        o = syn::align_up(o + syn::gemm_act_bytes(tpad, (int)hidden), 256);
        m.h = o;
        o = syn::align_up(o + 4ull * ent * inter, 256);
        m.hq = o;
        o = syn::align_up(o + syn::gemm_act_bytes(tpad, (int)inter), 256);
    } else {
        m.xq = o;
        o += syn::moe_act_bytes((int64_t)ent, (int)hidden);
        m.h = o;
        o = syn::align_up(o + 4ull * ent * inter, 256);
        m.hq = o;
        o += syn::moe_act_bytes((int64_t)ent, (int)inter);
    }
    m.bytes = syn::align_up(o, 256);
    return m;
}

// Q8_0 experts: the workspace after the packing's words: the entries' x rows in Q8_0 (codes
// [entries][hidden], scales [entries][hidden / 32]), h F32 [entries][inter], h in Q8_0.
struct MoeQ8Ws {
    uint64_t xq, xd, h, hq, hd, bytes;
};
MoeQ8Ws moe_q8_ws(const MoeWs& head, uint32_t top_k, uint32_t hidden, uint32_t inter, uint32_t rows) {
    MoeQ8Ws m{};
    const uint64_t ent = (uint64_t)rows * top_k;
    uint64_t o = head.xq;
    m.xq = o;
    o = syn::align_up(o + ent * hidden, 256);
    m.xd = o;
    o = syn::align_up(o + 4 * ent * (hidden / 32), 256);
    m.h = o;
    o = syn::align_up(o + 4 * ent * inter, 256);
    m.hq = o;
    o = syn::align_up(o + ent * inter, 256);
    m.hd = o;
    o = syn::align_up(o + 4 * ent * (inter / 32), 256);
    m.bytes = o;
    return m;
}

// The packing's words of the workspace (offsets, slots, the error word), as moe_ws lays them.
MoeWs moe_head(uint32_t n_experts, uint32_t top_k, uint32_t rows) {
    MoeWs m{};
    uint64_t o = 0;
    m.offsets = o;
    o = syn::align_up(o + 4ull * (n_experts + 1), 256);
    m.slots = o;
    o = syn::align_up(o + 4ull * rows * top_k, 256);
    m.err = o;
    o = syn::align_up(o + 8, 256);
    m.xq = o;
    return m;
}

int check_moe_shape(const char* W, uint32_t n_experts, uint32_t top_k, uint32_t hidden,
                    uint32_t inter, uint32_t rows, int32_t wtype = SYN_Q4_K) {
    if (n_experts == 0 || n_experts > 256) return fail(SYN_E_UNSUPPORTED, "%s: n_experts %u (1..256)", W, n_experts);
    if (top_k == 0 || top_k > n_experts || top_k > 32) return fail(SYN_E_UNSUPPORTED, "%s: top_k %u (1..min(n_experts, 32))", W, top_k);
    const uint32_t be = wtype == SYN_Q8_0 ? 32 : 256;
    if (hidden % be || inter % be || hidden == 0 || inter == 0)
        return fail(SYN_E_INVALID, "%s: hidden %u and inter %u must be whole %u-weight blocks", W, hidden, inter, be);
    if (hidden > 65536 || inter > 65536) return fail(SYN_E_UNSUPPORTED, "%s: hidden/inter above 65536", W);
    if ((uint64_t)rows * top_k > 65536) return fail(SYN_E_UNSUPPORTED, "%s: rows * top_k above 65536", W);
    // the expert kernels address the entries' codes with 32-bit offsets
    if ((uint64_t)rows * top_k * (hidden > inter ? hidden : inter) >= (1ull << 32))
        return fail(SYN_E_UNSUPPORTED, "%s: rows * top_k * max(hidden, inter) reaches 2^32", W);
    return SYN_OK;
}

}  // namespace

int syn_moe_route_rows(const float* router, const float* x, uint32_t rows, uint32_t hidden,
                             uint32_t n_experts, uint32_t top_k, int32_t renormalize,
                             int32_t* ids, float* w, float* probs, void* stream, const uint32_t* active) {
    const char* W = "syn_moe_route";
    if (n_experts == 0 || n_experts > 256) return fail(SYN_E_UNSUPPORTED, "%s: n_experts %u (1..256)", W, n_experts);
    if (top_k == 0 || top_k > n_experts || top_k > 32) return fail(SYN_E_UNSUPPORTED, "%s: top_k %u", W, top_k);
    if (hidden % 32 || hidden == 0 || hidden > 8192 || !syn::moe_route_supported((int)hidden))
        return fail(SYN_E_UNSUPPORTED, "%s: hidden %u (whole 32-blocks, at most 8192)", W, hidden);
    if (rows == 0) return SYN_OK;
    if (!router || !x || !ids || !w || !probs) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(router, 16) || !aligned(x, 4)) return fail(SYN_E_INVALID, "%s: router must be 16-byte aligned", W);
    // the logits are staged in probs, row by row, before the softmax overwrites them
    syn::launch_moe_route(router, x, (int)rows, (int)hidden, (int)n_experts, (int)top_k, renormalize != 0,
                          ids, w, probs, probs, (hipStream_t)stream, active);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_route(const float* router, const float* x, uint32_t rows, uint32_t hidden,
                             uint32_t n_experts, uint32_t top_k, int32_t renormalize,
                             int32_t* ids, float* w, float* probs, void* stream) {
    return syn_moe_route_rows(router, x, rows, hidden, n_experts, top_k, renormalize, ids, w, probs, stream, nullptr);
}

SYN_EXPORT int syn_moe_pack(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                            uint32_t* offsets, uint32_t* slots, uint32_t* err, void* stream) {
    const char* W = "syn_moe_pack";
    if (n_experts == 0 || n_experts > 256) return fail(SYN_E_UNSUPPORTED, "%s: n_experts %u (1..256)", W, n_experts);
    if ((uint64_t)rows * top_k > 65536) return fail(SYN_E_UNSUPPORTED, "%s: rows * top_k above 65536", W);
    if (!ids || !offsets || !slots || !err) return fail(SYN_E_INVALID, "%s: null operand", W);
    syn::launch_moe_pack(ids, (int)(rows * top_k), (int)n_experts, offsets, slots, err, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_grouped_workspace_bytes(int32_t wtype, uint32_t n_experts, uint32_t top_k,
                                               uint32_t hidden, uint32_t inter, uint32_t rows,
                                               uint64_t* bytes) {
    const char* W = "syn_moe_grouped_workspace_bytes";
    if (wtype != SYN_Q4_K && wtype != SYN_Q8_0)
        return fail(SYN_E_UNSUPPORTED, "%s: expert weight type %d (Q4_K or Q8_0)", W, wtype);
    if (int rc = check_moe_shape(W, n_experts, top_k, hidden, inter, rows, wtype)) return rc;
    if (!bytes) return fail(SYN_E_INVALID, "%s: null output", W);
    *bytes = wtype == SYN_Q8_0 ? moe_q8_ws(moe_head(n_experts, top_k, rows), top_k, hidden, inter, rows).bytes
                               : moe_ws(n_experts, top_k, hidden, inter, rows).bytes;
    return SYN_OK;
}

namespace {

// MoeGrouped over Q8_0 experts: pack, Q8_0 of the entries' rows, gate/up + silu, Q8_0 of h, down.
int moe_grouped_q8_0(const void* gate, const void* up, const void* down, uint64_t expert_bytes_each,
                     uint32_t n_experts, uint32_t top_k, uint32_t hidden, uint32_t inter, const float* x,
                     const int32_t* ids, const int32_t* site, uint32_t rows, float* out, void* ws, uint64_t ws_bytes,
                     uint32_t* status, void* stream, const uint32_t* active, uint32_t* report) {
    const char* W = "syn_moe_grouped";
    const uint64_t mat = (uint64_t)inter * (hidden / 32) * 34;  // gate/up; down is the same size
    if (expert_bytes_each < mat * n_experts)
        return fail(SYN_E_INVALID, "%s: each stacked matrix holds %llu bytes, the experts need %llu", W,
                    (unsigned long long)expert_bytes_each, (unsigned long long)(mat * n_experts));
    const MoeWs head = moe_head(n_experts, top_k, rows);
    const MoeQ8Ws m = moe_q8_ws(head, top_k, hidden, inter, rows);
    if (ws_bytes < m.bytes)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)m.bytes);
    if (!gate || !up || !down || !x || !ids || !out || !ws) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (site && !aligned(site, 4)) return fail(SYN_E_INVALID, "%s: the site mask must be 4-byte aligned", W);
    if (!aligned(gate, 2) || !aligned(up, 2) || !aligned(down, 2) || !aligned(x, 16) || !aligned(ws, 256) ||
        !aligned(out, 4))
        return fail(SYN_E_INVALID, "%s: x must be 16-byte, the workspace 256-byte aligned", W);
    uint8_t* base = (uint8_t*)ws;
    uint32_t* offsets = (uint32_t*)(base + head.offsets);
    uint32_t* slots = (uint32_t*)(base + head.slots);
    uint32_t* err = (uint32_t*)(base + head.err);
    const int ent = (int)(rows * top_k);
    hipStream_t st = (hipStream_t)stream;
    int8_t* xq = (int8_t*)(base + m.xq);
    float* xd = (float*)(base + m.xd);
    float* h = (float*)(base + m.h);
    int8_t* hq = (int8_t*)(base + m.hq);
    float* hd = (float*)(base + m.hd);
    syn::launch_moe_pack(ids, ent, (int)n_experts, offsets, slots, err, st, active, (int)top_k, site, report);
    syn::launch_moe_gather_q8_0(x, slots, ent, (int)top_k, (int)hidden, err, xq, xd, 1, offsets + n_experts, st);
    syn::launch_moe_q8(0, (const uint8_t*)gate, (const uint8_t*)up, mat, (int)n_experts, (int)inter, (int)hidden,
                       offsets, slots, err, xq, xd, h, st);
    syn::launch_moe_gather_q8_0(h, slots, ent, (int)top_k, (int)inter, err, hq, hd, 0, offsets + n_experts, st);
    syn::launch_moe_q8(1, (const uint8_t*)down, nullptr, mat, (int)n_experts, (int)hidden, (int)inter, offsets,
                       slots, err, hq, hd, out, st);
    if (status) {
        hipError_t e = hipMemcpyAsync(status, err, 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return fail(SYN_E_DEVICE, "%s: status copy: %s", W, hipGetErrorString(e));
    }
    return check_launch(W);
}

}  // namespace

int syn_moe_grouped_rows(int32_t wtype, const void* gate, const void* up, const void* down,
                               uint64_t expert_bytes_each, uint32_t n_experts, uint32_t top_k,
                               uint32_t hidden, uint32_t inter, const float* x, const int32_t* ids,
                               const int32_t* site, uint32_t rows, float* out, void* ws, uint64_t ws_bytes,
                               uint32_t* status, void* stream, const uint32_t* active, uint32_t* report,
                               uint32_t layout) {
    const char* W = "syn_moe_grouped";
    if (wtype != SYN_Q4_K && wtype != SYN_Q8_0)
        return fail(SYN_E_UNSUPPORTED, "%s: expert weight type %d (Q4_K or Q8_0)", W, wtype);
    if (layout != SYN_LAYOUT_SOURCE && !(layout == SYN_LAYOUT_TILE64 && wtype == SYN_Q4_K))
        return fail(SYN_E_UNSUPPORTED, "%s: experts of type %d in layout %u (0, or 3 for Q4_K)", W, wtype, layout);
    if (int rc = check_moe_shape(W, n_experts, top_k, hidden, inter, rows, wtype)) return rc;
    if (rows == 0) return SYN_OK;
    if (wtype == SYN_Q8_0)
        return moe_grouped_q8_0(gate, up, down, expert_bytes_each, n_experts, top_k, hidden, inter, x, ids, site,
                                rows, out, ws, ws_bytes, status, stream, active, report);
    const uint64_t mat = (uint64_t)inter * (hidden / 256) * 144;  // gate/up; down is the same size
    if (expert_bytes_each < mat * n_experts)
        return fail(SYN_E_INVALID, "%s: each stacked matrix holds %llu bytes, the experts need %llu", W,
                    (unsigned long long)expert_bytes_each, (unsigned long long)(mat * n_experts));
    const MoeWs m = moe_ws(n_experts, top_k, hidden, inter, rows);
    if (ws_bytes < m.bytes)
        return fail(SYN_E_WORKSPACE, "%s: the workspace holds %llu bytes, the call needs %llu", W,
                    (unsigned long long)ws_bytes, (unsigned long long)m.bytes);
    if (!gate || !up || !down || !x || !ids || !out || !ws) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (site && !aligned(site, 4)) return fail(SYN_E_INVALID, "%s: the site mask must be 4-byte aligned", W);
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(down, 16) || !aligned(x, 16) || !aligned(ws, 256) || !aligned(out, 4))
        return fail(SYN_E_INVALID, "%s: weights and x must be 16-byte, the workspace 256-byte aligned", W);
    uint8_t* base = (uint8_t*)ws;
    uint32_t* offsets = (uint32_t*)(base + m.offsets);
    uint32_t* slots = (uint32_t*)(base + m.slots);
    uint32_t* err = (uint32_t*)(base + m.err);
    const int ent = (int)(rows * top_k);
    hipStream_t st = (hipStream_t)stream;
    syn::launch_moe_pack(ids, ent, (int)n_experts, offsets, slots, err, st, active, (int)top_k, site, report);
    if (m.gemm) {
        const syn::MoeTiles mt{(uint32_t*)(base + m.pad_off), (uint32_t*)(base + m.tile_e),
                               (uint32_t*)(base + m.n_tiles)};
        const int64_t tpad = 64ll * m.max_tiles;
        // the tokens' rows quantized once (the gate/up stage gathers each position's token)
        const syn::GemmAct gx = syn::gemm_act_at(base + m.xq, (int64_t)syn::align_up(rows, 64), (int)hidden);
        const syn::GemmAct gh = syn::gemm_act_at(base + m.hq, tpad, (int)inter);
        float* h = (float*)(base + m.h);
        syn::launch_moe_tiles(offsets, (int)n_experts, err, mt, st);
        syn::launch_gemm_act(x, (int)rows, (int)hidden, gx, st, active);
        syn::launch_moe_gemm(0, (const uint8_t*)gate, (const uint8_t*)up, (int)n_experts, (int)inter, (int)hidden,
                             gx, m.max_tiles, offsets, mt, err, slots, h, st, (int)top_k, (int)layout);
        syn::launch_moe_gemm_act(h, (int)inter, offsets, mt, err, gh, st);
        syn::launch_moe_gemm(1, (const uint8_t*)down, nullptr, (int)n_experts, (int)hidden, (int)inter, gh,
                             m.max_tiles, offsets, mt, err, slots, out, st, (int)top_k, (int)layout);
        if (status) {
            hipError_t e = hipMemcpyAsync(status, err, 4, hipMemcpyDeviceToDevice, st);
            if (e != hipSuccess) return fail(SYN_E_DEVICE, "%s: status copy: %s", W, hipGetErrorString(e));
        }
        return check_launch(W);
    }
    const syn::MoeAct ax = syn::moe_act_at(base + m.xq, ent, (int)hidden);
    const syn::MoeAct ah = syn::moe_act_at(base + m.hq, ent, (int)inter);
    syn::launch_moe_gather_q8k(x, slots, ent, (int)top_k, (int)hidden, err, ax, 1, st, offsets + n_experts);
    float* h = (float*)(base + m.h);
    syn::launch_moe_gateup((const uint8_t*)gate, (const uint8_t*)up, (int)n_experts, (int)hidden, (int)inter,
                           offsets, ent, ax, err, h, st, (int)layout);
    syn::launch_moe_gather_q8k(h, slots, ent, (int)top_k, (int)inter, err, ah, 0, st, offsets + n_experts);
    syn::launch_moe_down((const uint8_t*)down, (int)n_experts, (int)hidden, (int)inter, offsets, ent, ah,
                         slots, err, out, st, (int)layout);
    if (status) {
        hipError_t e = hipMemcpyAsync(status, err, 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return fail(SYN_E_DEVICE, "%s: status copy: %s", W, hipGetErrorString(e));
    }
    return check_launch(W);
}

SYN_EXPORT int syn_moe_grouped(int32_t wtype, const void* gate, const void* up, const void* down,
                               uint64_t expert_bytes_each, uint32_t n_experts, uint32_t top_k,
                               uint32_t hidden, uint32_t inter, const float* x, const int32_t* ids,
                               const int32_t* site, uint32_t rows, float* out, void* ws, uint64_t ws_bytes,
                               uint32_t* status, void* stream) {
    return syn_moe_grouped_rows(wtype, gate, up, down, expert_bytes_each, n_experts, top_k, hidden, inter, x, ids,
                                site, rows, out, ws, ws_bytes, status, stream, nullptr);
}

SYN_EXPORT int syn_moe_grouped_layout(uint32_t layout, int32_t wtype, const void* gate, const void* up,
                                      const void* down, uint64_t expert_bytes_each, uint32_t n_experts,
                                      uint32_t top_k, uint32_t hidden, uint32_t inter, const float* x,
                                      const int32_t* ids, const int32_t* site, uint32_t rows, float* out, void* ws,
                                      uint64_t ws_bytes, uint32_t* status, void* stream) {
    return syn_moe_grouped_rows(wtype, gate, up, down, expert_bytes_each, n_experts, top_k, hidden, inter, x, ids,
                                site, rows, out, ws, ws_bytes, status, stream, nullptr, nullptr, layout);
}

int syn_moe_combine_rows(const float* out, const int32_t* ids, const float* w, uint32_t rows,
                               uint32_t top_k, uint32_t hidden, float* y, void* stream, const uint32_t* active) {
    const char* W = "syn_moe_combine";
    if (top_k == 0 || top_k > 64) return fail(SYN_E_UNSUPPORTED, "%s: top_k %u (1..64)", W, top_k);
    if (rows == 0 || hidden == 0) return SYN_OK;
    if (!out || !ids || !w || !y) return fail(SYN_E_INVALID, "%s: null operand", W);
    syn::launch_moe_combine(out, ids, w, (int)rows, (int)top_k, (int)hidden, y, (hipStream_t)stream, active);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_combine(const float* out, const int32_t* ids, const float* w, uint32_t rows,
                               uint32_t top_k, uint32_t hidden, float* y, void* stream) {
    return syn_moe_combine_rows(out, ids, w, rows, top_k, hidden, y, stream, nullptr);
}

int syn_moe_combine_ranked_rows(const float* out, const float* w, uint32_t n_shared, const float* const* shared,
                                uint32_t rows, uint32_t top_k, uint32_t hidden, float* y, void* stream,
                                const uint32_t* active) {
    const char* W = "syn_moe_combine_ranked";
    if (top_k == 0 || top_k > 64) return fail(SYN_E_UNSUPPORTED, "%s: top_k %u (1..64)", W, top_k);
    if (n_shared > (uint32_t)syn::MAX_SHARED)
        return fail(SYN_E_UNSUPPORTED, "%s: %u shared experts (at most %d)", W, n_shared, syn::MAX_SHARED);
    if (rows == 0 || hidden == 0) return SYN_OK;
    if (!out || !w || !y || (n_shared && !shared)) return fail(SYN_E_INVALID, "%s: null operand", W);
    syn::SharedOuts sh{};
    sh.n = (int)n_shared;
    for (uint32_t i = 0; i < n_shared; ++i) {
        if (!shared[i]) return fail(SYN_E_INVALID, "%s: null shared output %u", W, i);
        sh.p[i] = shared[i];
    }
    syn::launch_moe_combine_ranked(out, w, sh, (int)rows, (int)top_k, (int)hidden, y, (hipStream_t)stream, active);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_combine_ranked(const float* out, const float* w, uint32_t n_shared,
                                      const float* const* shared, uint32_t rows, uint32_t top_k, uint32_t hidden,
                                      float* y, void* stream) {
    return syn_moe_combine_ranked_rows(out, w, n_shared, shared, rows, top_k, hidden, y, stream, nullptr);
}

// ============================================================================================
// The residency split
// ============================================================================================

SYN_EXPORT int syn_moe_doorbell(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                                const uint32_t* slot_of, const void* step_desc, uint32_t seq, void* layer,
                                uint32_t max_union, uint32_t* status, void* stream) {
    const char* W = "syn_moe_doorbell";
    if (n_experts == 0 || n_experts > 8192) return fail(SYN_E_UNSUPPORTED, "%s: n_experts %u (1..8192)", W, n_experts);
    if (top_k == 0 || top_k > 32) return fail(SYN_E_UNSUPPORTED, "%s: top_k %u (1..32)", W, top_k);
    if (rows > 65535) return fail(SYN_E_UNSUPPORTED, "%s: %u rows; a route entry counts at most 65535 tokens", W, rows);
    if (max_union > 65535) return fail(SYN_E_INVALID, "%s: max_union %u above 65535", W, max_union);
    if (!layer || (rows && !ids)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(layer, 8) || !aligned(step_desc, 8))
        return fail(SYN_E_INVALID, "%s: the layer and the step descriptor must be 8-byte aligned", W);
    syn::launch_moe_doorbell(ids, (int)rows, (int)top_k, (int)n_experts, slot_of, step_desc, seq, (uint8_t*)layer,
                             max_union, status, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_assign(const void* route, uint32_t n_route, const uint32_t* eligible, uint32_t n_experts,
                              uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots, uint32_t* out,
                              void* stream) {
    const char* W = "syn_moe_assign";
    if (n_route > 65535) return fail(SYN_E_INVALID, "%s: %u route entries; a doorbell holds at most 65535", W, n_route);
    if (n_route == 0) return SYN_OK;
    if (!route || !out || (n_experts && !eligible)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(route, 8) || !aligned(out, 4) || !aligned(eligible, 4))
        return fail(SYN_E_INVALID, "%s: the route entries must be 8-byte aligned", W);
    syn::launch_moe_assign((const uint8_t*)route, n_route, eligible, n_experts, b_copy, expert_bytes, copy_slots,
                           out, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_assign_layer(const void* layer, uint32_t max_union, const uint32_t* eligible,
                                    uint32_t n_experts, const uint32_t* b_copy, uint64_t expert_bytes,
                                    uint32_t copy_slots, uint32_t* out, void* stream) {
    const char* W = "syn_moe_assign_layer";
    if (max_union > 65535) return fail(SYN_E_INVALID, "%s: max_union %u above 65535", W, max_union);
    if (!layer || !b_copy || (max_union && !out) || (n_experts && !eligible))
        return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(layer, 8) || !aligned(b_copy, 4) || !aligned(out, 4) || !aligned(eligible, 4))
        return fail(SYN_E_INVALID, "%s: the layer must be 8-byte aligned", W);
    syn::launch_moe_assign_layer((const uint8_t*)layer, max_union, eligible, n_experts, b_copy, expert_bytes,
                                 copy_slots, out, (hipStream_t)stream);
    return check_launch(W);
}

SYN_EXPORT int syn_moe_site_mask(const void* layer, uint32_t max_union, const uint32_t* codes, uint32_t n_experts,
                                 int32_t which, int32_t* site, void* stream) {
    const char* W = "syn_moe_site_mask";
    if (which < 0 || which > 2) return fail(SYN_E_INVALID, "%s: class %d (0 HIT, 1 COPY, 2 CPU)", W, which);
    if (max_union > 65535) return fail(SYN_E_INVALID, "%s: max_union %u above 65535", W, max_union);
    if (n_experts == 0) return SYN_OK;
    if (!layer || !site || (max_union && !codes)) return fail(SYN_E_INVALID, "%s: null operand", W);
    if (!aligned(layer, 8) || !aligned(codes, 4) || !aligned(site, 4))
        return fail(SYN_E_INVALID, "%s: the layer must be 8-byte aligned", W);
    syn::launch_moe_site_mask((const uint8_t*)layer, max_union, codes, (int)n_experts, which, site,
                              (hipStream_t)stream);
    return check_launch(W);
}
