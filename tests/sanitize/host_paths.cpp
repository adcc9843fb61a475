// The host-side code of both libraries under AddressSanitizer and UndefinedBehaviorSanitizer:
// every path a host without a GPU reaches.  Built with clang's sanitizers against libraries
// whose host code is instrumented (the kernels' device code is not), and run by
// tests/test_host_sanitizers.py; any sanitizer report, or a failed check, fails the run.
//
// Covered: the provider's entry handshake, its JSON reader on valid and mutated OpKeys (through
// repack / repacked_len, which parse a key without a context), repack of every served layout,
// the out-buffer protocol of build / enumerate / ops, the refusals of an unknown context and of
// open without a device, per-thread messages; the C API's workspace sizing over extreme shapes,
// the host repacks (round trips, and bytes equal to the provider's), and argument refusals.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/syntropy_hip.h"
#include "../../include/syntropy_provider.h"

static int g_fails = 0;
#define CHECK(c)                                                             \
    do {                                                                     \
        if (!(c)) {                                                          \
            std::fprintf(stderr, "check failed, line %d: %s\n", __LINE__, #c); \
            ++g_fails;                                                       \
        }                                                                    \
    } while (0)

static void host_log(uint8_t, const char*, const char*, size_t) {}
static void host_metric(uint32_t, uint64_t) {}
static const char* host_config(const char* key) {
    // a spin bound that is not a number: the provider must not read past it or overflow
    if (!std::strcmp(key, "kernels.spin_kernel_max_us")) return "99999999999999999999";
    return nullptr;
}

static SynHostApi host_api() {
    SynHostApi h{};
    std::memcpy(h.h.magic, SYN_PROVIDER_MAGIC, 8);
    h.h.abi_major = SYN_ABI_MAJOR;
    h.h.abi_minor = SYN_ABI_MINOR;
    h.h.struct_size = sizeof(SynHostApi);
    h.log = host_log;
    h.metric = host_metric;
    h.config = host_config;
    return h;
}

static std::string key(const char* op, const char* weight, int layout = 0) {
    std::string s = std::string("{\"op\":") + op + ",\"schemes\":[";
    if (weight) s += std::string("{\"Ggml\":\"") + weight + "\"},";
    s += "{\"Plain\":\"F32\"},{\"Plain\":\"F32\"}],\"layout\":" + std::to_string(layout) + ",\"variant\":0}";
    return s;
}

static std::string message(const SynProviderVtbl* v) {
    size_t len = 0;
    v->last_error(v->slf, 0, nullptr, 0, &len);
    std::vector<uint8_t> b(len + 1, 0);
    v->last_error(v->slf, 0, b.data(), b.size(), &len);
    return std::string(reinterpret_cast<const char*>(b.data()), len < b.size() ? len : b.size());
}

// the out-buffer protocol: a short buffer gets the length only, then the whole text
static std::string outbuf(const SynProviderVtbl* v, SynStatus (*fn)(void*, SynOutBuf*)) {
    SynOutBuf o{nullptr, 0, 0};
    CHECK(fn(v->slf, &o).cls == SYN_CLASS_OK);
    std::vector<uint8_t> b(o.len);
    SynOutBuf p{b.data(), b.size(), 0};
    CHECK(fn(v->slf, &p).cls == SYN_CLASS_OK);
    CHECK(p.len == b.size());
    return std::string(b.begin(), b.end());
}

static void provider_paths() {
    CHECK(syntropy_provider_entry_v1(nullptr) == nullptr);
    SynHostApi bad = host_api();
    bad.h.magic[0] = 'X';
    CHECK(syntropy_provider_entry_v1(&bad) == nullptr);
    bad = host_api();
    bad.h.abi_major = 2;
    CHECK(syntropy_provider_entry_v1(&bad) == nullptr);
    bad = host_api();
    bad.h.struct_size = sizeof(SynHostApi) - 1;
    CHECK(syntropy_provider_entry_v1(&bad) == nullptr);

    const SynHostApi h = host_api();
    const SynModule* m = syntropy_provider_entry_v1(&h);
    CHECK(m && m->n_providers == 1);
    if (!m) return;
    const SynProviderVtbl* v = m->providers;
    CHECK(std::string(v->id) == "hip");

    CHECK(outbuf(v, v->build).find('{') == 0);
    CHECK(outbuf(v, v->ops).find("Gemv") != std::string::npos);
    (void)outbuf(v, v->enumerate);

    // no device here: open refuses, an unknown context is refused, messages are per thread
    uint64_t ctx = 0;
    SynDeviceId dev{};
    SynOpenOptions opts{};
    CHECK(v->open(v->slf, &dev, &opts, &ctx).cls != SYN_CLASS_OK);
    CHECK(!message(v).empty());
    const std::string q = key("\"Gemv\"", "Q4_K");
    const std::string shape = "{\"rows\":1,\"dims\":[4096,4096]}";
    SynOutBuf o{nullptr, 0, 0};
    CHECK(v->query(v->slf, 987654, reinterpret_cast<const uint8_t*>(q.data()), q.size(),
                   reinterpret_cast<const uint8_t*>(shape.data()), shape.size(), &o).cls != SYN_CLASS_OK);
    const std::string mine = message(v);
    std::thread([&] { CHECK(message(v) != mine || mine.empty()); }).join();
    SynHealth hl{};
    CHECK(v->health(v->slf, 987654, &hl).cls == SYN_CLASS_OK && hl.kind == 0);  // module-wide, healthy
    CHECK(v->close_ctx(v->slf, 987654).cls != SYN_CLASS_OK);
    uint64_t s = 0;
    CHECK(v->stream(v->slf, 987654, 0, &s).cls != SYN_CLASS_OK);

    // repack of every served layout, and the refusals of wrong lengths
    std::mt19937_64 rng(7);
    struct Case { const char* w; size_t block; uint32_t layout; };
    const Case cases[] = {{"Q4_K", 144, 1}, {"Q8_0", 34, 2}, {"Q4_0", 18, 2}};
    const char* ops[] = {"\"Gemv\"", "\"Gemm\"", "\"Logits\"", "{\"GateUpAct\":{\"act\":\"Silu\"}}"};
    for (const Case& c : cases)
        for (const char* op : ops)
            for (size_t nblk : {size_t(0), size_t(1), size_t(7), size_t(8), size_t(9), size_t(67)}) {
                const std::string k = key(op, c.w);
                const auto* kb = reinterpret_cast<const uint8_t*>(k.data());
                std::vector<uint8_t> src(nblk * c.block), dst(src.size() + 1, 0xEE);
                for (auto& b : src) b = (uint8_t)rng();
                uint32_t present = 7, layout = 7;
                uint64_t n = 7;
                CHECK(v->repacked_len(v->slf, kb, k.size(), src.size(), &present, &n).cls == SYN_CLASS_OK);
                CHECK(present == 1 && n == src.size());
                CHECK(v->repack(v->slf, kb, k.size(), src.data(), src.size(), dst.data(), src.size(), &present,
                                &layout).cls == SYN_CLASS_OK);
                CHECK(present == 1 && layout == c.layout);
                CHECK(dst[src.size()] == 0xEE);  // nothing written past dst_len
                // the C API's host repack gives the same bytes, and its inverse the source
                std::vector<uint8_t> viaapi(src.size()), back(src.size());
                const int wt = c.block == 144 ? SYN_Q4_K : c.block == 34 ? SYN_Q8_0 : SYN_Q4_0;
                const int r1 = c.block == 144 ? syn_q4k_repack_host(c.layout, src.data(), viaapi.data(), src.size(), 0)
                                              : syn_split_repack_host(c.layout, wt, src.data(), viaapi.data(), src.size(), 0);
                const int r2 = c.block == 144 ? syn_q4k_repack_host(c.layout, viaapi.data(), back.data(), src.size(), 1)
                                              : syn_split_repack_host(c.layout, wt, viaapi.data(), back.data(), src.size(), 1);
                CHECK(r1 == 0 && r2 == 0);
                CHECK(src.empty() || std::memcmp(viaapi.data(), dst.data(), src.size()) == 0);
                CHECK(back == src);
                if (nblk) {
                    CHECK(v->repack(v->slf, kb, k.size(), src.data(), src.size() - 1, dst.data(), dst.size(),
                                    &present, &layout).cls == SYN_CLASS_INVALID_REQUEST);
                    CHECK(v->repack(v->slf, kb, k.size(), src.data(), src.size(), dst.data(), src.size() - 1,
                                    &present, &layout).cls == SYN_CLASS_INVALID_REQUEST);
                }
            }

    // the JSON reader on mutated keys: truncations, byte flips, insertions, deep nesting, long
    // strings.  Any status is acceptable; reading outside the key is not.
    std::vector<std::string> seeds;
    for (const Case& c : cases)
        for (const char* op : ops) seeds.push_back(key(op, c.w));
    seeds.push_back(key("{\"MoeRoute\":{\"norm\":\"Softmax\"}}", nullptr));
    seeds.push_back(key("\"MoeGrouped\"", "Q4_K"));
    seeds.push_back(std::string(40, '[') + std::string(40, ']'));
    seeds.push_back("{\"op\":\"" + std::string(5000, 'G') + "\"}");
    seeds.push_back("{\"layout\":1e400,\"variant\":-0,\"op\":\"Gemv\",\"schemes\":[]}");
    seeds.push_back("{\"op\":\"Gemv\\");
    const char alphabet[] = "{}[]\":,\\ 0123456789-+.eE\ttruefalsenullGgmlPlainF32Q4_K";
    std::vector<uint8_t> src(144 * 9), dst(144 * 9);
    for (int it = 0; it < 40000; ++it) {
        std::string k = seeds[rng() % seeds.size()];
        const int edits = 1 + (int)(rng() % 4);
        for (int e = 0; e < edits && !k.empty(); ++e) {
            const size_t at = rng() % k.size();
            switch (rng() % 4) {
                case 0: k.resize(at); break;
                case 1: k[at] = (char)rng(); break;
                case 2: k.insert(k.begin() + at, alphabet[rng() % (sizeof(alphabet) - 1)]); break;
                default: k.erase(k.begin() + at); break;
            }
        }
        // the key in a buffer of exactly its size, so that a read past it is caught
        std::vector<uint8_t> kb(k.begin(), k.end());
        uint32_t present = 0, layout = 0;
        uint64_t n = 0;
        const SynStatus a = v->repacked_len(v->slf, kb.data(), kb.size(), src.size(), &present, &n);
        const SynStatus b = v->repack(v->slf, kb.data(), kb.size(), src.data(), src.size(), dst.data(), dst.size(),
                                      &present, &layout);
        CHECK(a.cls == SYN_CLASS_OK || a.cls == SYN_CLASS_INVALID_REQUEST || a.cls == SYN_CLASS_UNSUPPORTED);
        CHECK(b.cls == SYN_CLASS_OK || b.cls == SYN_CLASS_INVALID_REQUEST || b.cls == SYN_CLASS_UNSUPPORTED);
    }
}

static void capi_paths() {
    CHECK(syn_version() > 0);
    const int32_t types[] = {-1, 0, SYN_F16, SYN_Q4_0, SYN_Q8_0, SYN_Q4_K, SYN_BF16, 1000};
    const uint32_t rows[] = {0u, 1u, 8u, 9u, 65535u, 0x7FFFFFFFu, 0xFFFFFFFFu};
    const uint32_t ks[] = {0u, 32u, 255u, 256u, 4096u, 14336u, 0x80000000u, 0xFFFFFF00u, 0xFFFFFFFFu};
    uint64_t bytes = 0;
    for (int32_t t : types)
        for (uint32_t r : rows)
            for (uint32_t k : ks) {
                (void)syn_gemv_workspace_bytes(t, r, k, &bytes);
                for (uint32_t layout : {0u, 1u, 2u, 9u}) {
                    (void)syn_gemv_layout_workspace_bytes(layout, t, r, k, &bytes);
                    (void)syn_gate_up_act_workspace_bytes(layout, t, r, k, k, &bytes);
                    (void)syn_logits_workspace_bytes(layout, t, r, k, k, &bytes);
                }
                (void)syn_gemm_workspace_bytes(r, k, &bytes);
                for (uint32_t e : {0u, 1u, 128u, 0xFFFFFFFFu})
                    (void)syn_moe_grouped_workspace_bytes(t, e, 8, k, k / 2, r, &bytes);
                (void)syn_gemv_batch_workspace_bytes(1, &k, &bytes);
            }
    CHECK(syn_gemv_workspace_bytes(SYN_Q4_K, 1, 4096, nullptr) != 0);
    CHECK(syn_gemv_workspace_bytes(SYN_Q4_K, 1, 4096, &bytes) == 0 && bytes > 0);
    CHECK(syn_gemv_batch_workspace_bytes(0, nullptr, &bytes) != 0 || bytes == 0);

    // host repacks: lengths that are not whole blocks, null pointers, unknown layouts
    std::vector<uint8_t> a(144 * 3), b(144 * 3);
    CHECK(syn_q4k_repack_host(1, a.data(), b.data(), 100, 0) != 0);
    CHECK(syn_q4k_repack_host(7, a.data(), b.data(), a.size(), 0) != 0);
    CHECK(syn_q4k_repack_host(1, nullptr, b.data(), a.size(), 0) != 0);
    CHECK(syn_split_repack_host(2, SYN_Q8_0, a.data(), b.data(), 33, 0) != 0);
    CHECK(syn_split_repack_host(2, SYN_Q4_K, a.data(), b.data(), 144, 0) != 0);
    CHECK(syn_split_repack_host(2, SYN_Q4_0, a.data(), nullptr, 18, 0) != 0);
    CHECK(std::strlen(syn_last_error()) > 0);

    // TILE64: two runs of 64 rows of 3 super-blocks; block b of row r lands at 144 (64 b + r)
    // of its run, and the inverse restores the rows
    {
        const uint32_t k = 768;
        const size_t rb = 3 * 144, bytes = 128 * rb;
        std::vector<uint8_t> src(bytes), t(bytes), back(bytes);
        std::mt19937_64 r64(11);
        for (auto& v : src) v = (uint8_t)r64();
        CHECK(syn_q4k_tile64_repack_host(src.data(), t.data(), bytes, k, 0) == 0);
        bool placed = true;
        for (size_t row = 0; row < 128; ++row)
            for (size_t blk = 0; blk < 3; ++blk)
                placed = placed && std::memcmp(t.data() + (row / 64) * 64 * rb + 144 * (64 * blk + row % 64),
                                               src.data() + row * rb + 144 * blk, 144) == 0;
        CHECK(placed);
        CHECK(syn_q4k_tile64_repack_host(t.data(), back.data(), bytes, k, 1) == 0 && back == src);
        CHECK(syn_q4k_tile64_repack_host(src.data(), t.data(), bytes - rb, k, 0) != 0);  // 127 rows
        CHECK(syn_q4k_tile64_repack_host(src.data(), t.data(), bytes, 700, 0) != 0);
        CHECK(syn_q4k_tile64_repack_host(src.data(), src.data(), bytes, k, 0) != 0);
        CHECK(syn_q4k_tile64_repack_host(nullptr, t.data(), bytes, k, 0) != 0);
        float xs[256] = {};
        CHECK(syn_moe_grouped_layout(3, SYN_Q8_0, a.data(), a.data(), a.data(), 0, 4, 2, 256, 256, xs,
                                     nullptr, nullptr, 1, nullptr, nullptr, 0, nullptr, nullptr) != 0);
        CHECK(syn_moe_grouped_layout(1, SYN_Q4_K, a.data(), a.data(), a.data(), 0, 4, 2, 256, 256, xs,
                                     nullptr, nullptr, 1, nullptr, nullptr, 0, nullptr, nullptr) != 0);
    }

    // the device entry points refuse malformed arguments (on a host without a GPU, or before
    // any launch): they must return an error, not read the null buffers
    float y[4];
    CHECK(syn_gemv(SYN_Q4_K, nullptr, 144, 1, 256, nullptr, 1, y, nullptr, 0, nullptr) != 0);
    CHECK(syn_gemv(SYN_Q4_K, a.data(), 100, 1, 256, y, 1, y, nullptr, 0, nullptr) != 0);
    CHECK(syn_gemv_layout(9, SYN_Q4_K, a.data(), 144, 1, 256, y, 1, y, nullptr, 0, nullptr) != 0);
    CHECK(syn_quantize(SYN_Q4_K, nullptr, 256, nullptr, 0, nullptr) != 0);
    CHECK(syn_dequantize(1000, a.data(), a.size(), y, nullptr) != 0);
}

int main() {
    provider_paths();
    capi_paths();
    if (g_fails) {
        std::fprintf(stderr, "%d checks failed\n", g_fails);
        return 1;
    }
    std::printf("host paths: all checks passed\n");
    return 0;
}
