// The provider-library boundary for MI355X: syntropy_provider_entry_v1 and its "hip" provider
// (include/syntropy_provider.h).  The reference's module side is crates/kernels/src/abi/
// (guest.rs: the thunks, export.rs: the table); its host side, kernels_loader::ModuleProvider
// (crates/kernels-loader/src/provider.rs), calls this table unchanged.
//
// Behaviour kept from the reference's guest:
//  * every entry runs under a catch-all; a caught exception returns Internal / ProviderPanicked
//    (16) and makes the provider sticky, after which every entry but health, free and close_ctx
//    returns Device / DeviceSticky (8) (guest.rs:184-230);
//  * the message of the last failure is kept per thread and read with last_error
//    (guest.rs:240-265);
//  * a context lives in a per-thread table: a handle used on another thread is refused
//    (guest.rs:267-280);
//  * query answers with CapsWire JSON or nothing (len 0) for an op it does not serve
//    (wire.rs:762-830); the JSON it reads is serde's form of OpKey and ShapeSig.
//
//  * a sticky device error (an illegal address, a failed launch and the like, RFC-0040 ...md:861,
//    933) seen by any entry makes the provider sticky with DeviceSticky (8);
//  * the core's host services (crates/kernels/src/abi/types.rs:47-58) are kept: `config` gives
//    kernels.spin_kernel_max_us at open and the fault-injection keys fixture.panic_in and
//    fixture.device_fault_in (read once, when the entry symbol is called; the names follow the
//    reference's test provider, crates/kernels-loader/examples/test_provider.rs:7-16), and `log`
//    receives every failure that makes the provider sticky or that the device reports later (a
//    doorbell timeout, a refused MoeGrouped).  The reference defines no metric ids for
//    providers, so `metric` is not called.
//
// The hot entries (launch, record, wait, poll, copy, copy_batch, replay, health) take no lock
// and allocate nothing: they look up handles in the calling thread's context and enqueue.
#include <hip/hip_runtime.h>
#include <linux/futex.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <atomic>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <exception>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/syntropy_hip.h"
#include "../../include/syntropy_provider.h"
#include "capi_rows.hpp"
#include "kernels.hpp"

#define SYN_PROVIDER_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

// ============================================================================================
// Status, messages, stickiness
// ============================================================================================

struct Fail {
    uint32_t cls;
    uint16_t code;
    std::string msg;
};

thread_local std::string t_message;
std::atomic<uint16_t> g_sticky{0};

// The core's services, copied when the entry symbol is called, and the fault-injection keys.
struct HostServices {
    SynHostApi api{};
    bool present = false;
    std::string panic_in;         // fixture.panic_in: the entry that throws
    std::string device_fault_in;  // fixture.device_fault_in: the entry that meets a sticky device error
};
HostServices g_host;
std::once_flag g_host_once;

const char* host_config(const char* key) {
    return g_host.present && g_host.api.config ? g_host.api.config(key) : nullptr;
}

// level: 0 error, 1 warn, 2 info (types.rs:50-52)
void host_log(uint8_t level, const std::string& msg) {
    if (g_host.present && g_host.api.log) g_host.api.log(level, "syntropy_amd::hip", msg.data(), msg.size());
}

SynStatus status(uint32_t cls, uint16_t code) {
    SynStatus s;
    s.cls = cls;
    s.domain = SYN_DOMAIN_KERNELS;
    s.code = code;
    s.retry = 0;
    return s;
}
const SynStatus OK = status(SYN_CLASS_OK, 0);

[[noreturn]] void fail(uint32_t cls, uint16_t code, std::string msg) { throw Fail{cls, code, std::move(msg)}; }
[[noreturn]] void internal(std::string msg) { fail(SYN_CLASS_INTERNAL, 0, std::move(msg)); }
[[noreturn]] void unsupported(std::string msg) { fail(SYN_CLASS_UNSUPPORTED, SYN_CODE_OP_UNSUPPORTED, std::move(msg)); }

// Errors after which the device cannot run further work in this process.
bool sticky_error(hipError_t e) {
    switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorPriorLaunchFailure:
    case hipErrorAssert:
    case hipErrorLaunchTimeOut:
    case hipErrorECCNotCorrectable:
        return true;
    default:
        return false;
    }
}

void check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    if (sticky_error(e)) {
        uint16_t none = 0;
        g_sticky.compare_exchange_strong(none, SYN_CODE_DEVICE_STICKY, std::memory_order_acq_rel);
        msg += " (the device is lost to this process: the provider is sticky)";
        host_log(0, msg);
        fail(SYN_CLASS_DEVICE, SYN_CODE_DEVICE_STICKY, std::move(msg));
    }
    fail(SYN_CLASS_DEVICE, 0, std::move(msg));
}
void check_syn(int rc, const char* what) {
    if (rc == SYN_OK) return;
    const std::string m = std::string(what) + ": " + syn_last_error();
    if (rc == SYN_E_UNSUPPORTED) unsupported(m);
    if (rc == SYN_E_WORKSPACE) fail(SYN_CLASS_INTERNAL, SYN_CODE_WORKSPACE_EXCEEDED, m);
    if (rc == SYN_E_DEVICE) fail(SYN_CLASS_DEVICE, 0, m);
    internal(m);
}

// Runs one entry: the sticky gate, the catch-all, the per-thread message.
template <class F>
SynStatus call(const char* name, bool allowed_when_sticky, F&& f) {
    const uint16_t sticky = g_sticky.load(std::memory_order_acquire);
    if (sticky && !allowed_when_sticky) {
        t_message = std::string("`") + name + "` refused: the provider is sticky after code " +
                    std::to_string(sticky);
        return status(SYN_CLASS_DEVICE, SYN_CODE_DEVICE_STICKY);
    }
    try {
        if (!g_host.panic_in.empty() && g_host.panic_in == name)
            throw std::runtime_error("injected by fixture.panic_in");
        if (!g_host.device_fault_in.empty() && g_host.device_fault_in == name)
            check_hip(hipErrorIllegalAddress, "injected by fixture.device_fault_in");
        f();
        return OK;
    } catch (const Fail& e) {
        t_message = e.msg;
        return status(e.cls, e.code);
    } catch (const std::exception& e) {
        g_sticky.store(SYN_CODE_PROVIDER_PANICKED, std::memory_order_release);
        t_message = std::string("the provider failed in `") + name + "`: " + e.what();
        host_log(0, t_message);
        return status(SYN_CLASS_INTERNAL, SYN_CODE_PROVIDER_PANICKED);
    } catch (...) {
        g_sticky.store(SYN_CODE_PROVIDER_PANICKED, std::memory_order_release);
        t_message = std::string("the provider failed in `") + name + "` with an unknown exception";
        host_log(0, t_message);
        return status(SYN_CLASS_INTERNAL, SYN_CODE_PROVIDER_PANICKED);
    }
}

void put(SynOutBuf* out, const std::string& s) {
    if (!out) internal("null output buffer");
    out->len = s.size();
    if (s.size() <= out->cap && out->ptr) std::memcpy(out->ptr, s.data(), s.size());
}

// ============================================================================================
// JSON: the serde forms of OpKey and ShapeSig (a small reader; objects keep their order)
// ============================================================================================

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const char* key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct Reader {
    const char* p;
    const char* end;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    [[noreturn]] void bad(const char* what) { fail(SYN_CLASS_INVALID_REQUEST, 0, std::string("JSON: ") + what); }
    std::string string() {
        if (p >= end || *p != '"') bad("expected a string");
        ++p;
        std::string s;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (p >= end) bad("unterminated escape");
                const char c = *p;
                s.push_back(c == 'n' ? '\n' : c == 't' ? '\t' : c == 'r' ? '\r' : c);
                if (c == 'u') bad("\\u escapes are not used by these records");
            } else {
                s.push_back(*p);
            }
            ++p;
        }
        if (p >= end) bad("unterminated string");
        ++p;
        return s;
    }
    Json value(int depth = 0) {
        if (depth > 32) bad("nested too deeply");
        ws();
        if (p >= end) bad("unexpected end");
        Json v;
        if (*p == '{') {
            ++p;
            v.kind = Json::Obj;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return v;
            }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= end || *p != ':') bad("expected ':'");
                ++p;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return v;
                }
                bad("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            ++p;
            v.kind = Json::Arr;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return v;
            }
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return v;
                }
                bad("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.kind = Json::Str;
            v.str = string();
            return v;
        }
        if (end - p >= 4 && !std::strncmp(p, "true", 4)) {
            p += 4;
            v.kind = Json::Bool;
            v.b = true;
            return v;
        }
        if (end - p >= 5 && !std::strncmp(p, "false", 5)) {
            p += 5;
            v.kind = Json::Bool;
            return v;
        }
        if (end - p >= 4 && !std::strncmp(p, "null", 4)) {
            p += 4;
            return v;
        }
        const char* s = p;
        while (p < end && (std::strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) ++p;
        if (p == s) bad("unexpected character");
        v.kind = Json::Num;
        v.num = std::strtod(std::string(s, p).c_str(), nullptr);
        return v;
    }
};

Json parse(const uint8_t* data, size_t len) {
    if (!data && len) internal("null JSON");
    Reader r{reinterpret_cast<const char*>(data), reinterpret_cast<const char*>(data) + len};
    Json v = r.value();
    r.ws();
    if (r.p != r.end) r.bad("trailing bytes");
    return v;
}

uint32_t u32_of(const Json* v, const char* what) {
    if (!v || v->kind != Json::Num || v->num < 0 || v->num > 4294967295.0 || v->num != (double)(uint64_t)v->num)
        fail(SYN_CLASS_INVALID_REQUEST, 0, std::string("JSON: ") + what + " must be an unsigned integer");
    return (uint32_t)v->num;
}

// ============================================================================================
// Ops served: keys, shapes, capabilities
// ============================================================================================

// Gemv, Gemm and Logits share one binding (a matrix product: the ggml provider maps all three
// to mul_mat, crates/kernels-ggml/src/mapping.rs:30); GateUpAct{Silu} takes the stacked
// [gate; up] weight (:31).
enum class Op { Gemv, Gemm, Logits, GateUpAct, MoeGrouped, MoeRoute, MoeCombine, Other };

bool dense(Op op) { return op == Op::Gemv || op == Op::Gemm || op == Op::Logits || op == Op::GateUpAct; }

struct Key {
    Op op = Op::Other;
    bool softmax = false;       // MoeRoute's norm
    bool silu = false;          // GateUpAct's act
    int weight = -1;            // ggml type id of schemes[0] when it is a Ggml scheme
    bool rest_plain_f32 = true;  // every other scheme is Plain(F32)
    size_t n_schemes = 0;
    uint32_t layout = 0, variant = 0;
};

int ggml_id(const std::string& name) {
    if (name == "F16") return SYN_F16;
    if (name == "BF16") return SYN_BF16;
    if (name == "Q4_0") return SYN_Q4_0;
    if (name == "Q8_0") return SYN_Q8_0;
    if (name == "Q4_K") return SYN_Q4_K;
    return -2;  // a ggml type this provider does not compute
}

Key parse_key(const uint8_t* data, size_t len) {
    const Json j = parse(data, len);
    if (j.kind != Json::Obj) fail(SYN_CLASS_INVALID_REQUEST, 0, "OpKey: not an object");
    Key k;
    const Json* op = j.get("op");
    if (!op) fail(SYN_CLASS_INVALID_REQUEST, 0, "OpKey: no op");
    if (op->kind == Json::Str) {
        if (op->str == "Gemv") k.op = Op::Gemv;
        else if (op->str == "Gemm") k.op = Op::Gemm;
        else if (op->str == "Logits") k.op = Op::Logits;
        else if (op->str == "MoeGrouped") k.op = Op::MoeGrouped;
        else if (op->str == "MoeCombine") k.op = Op::MoeCombine;
    } else if (op->kind == Json::Obj && op->obj.size() == 1 && op->obj[0].first == "MoeRoute") {
        k.op = Op::MoeRoute;
        const Json* norm = op->obj[0].second.get("norm");
        k.softmax = norm && norm->kind == Json::Str && norm->str == "Softmax";
    } else if (op->kind == Json::Obj && op->obj.size() == 1 && op->obj[0].first == "GateUpAct") {
        k.op = Op::GateUpAct;
        const Json* act = op->obj[0].second.get("act");
        k.silu = act && act->kind == Json::Str && act->str == "Silu";
    }
    const Json* schemes = j.get("schemes");
    if (!schemes || schemes->kind != Json::Arr) fail(SYN_CLASS_INVALID_REQUEST, 0, "OpKey: no schemes");
    k.n_schemes = schemes->arr.size();
    for (size_t i = 0; i < schemes->arr.size(); ++i) {
        const Json& s = schemes->arr[i];
        const bool plain_f32 = s.kind == Json::Obj && s.obj.size() == 1 && s.obj[0].first == "Plain" &&
                               s.obj[0].second.kind == Json::Str && s.obj[0].second.str == "F32";
        const bool plain = s.kind == Json::Obj && s.obj.size() == 1 && s.obj[0].first == "Plain" &&
                           s.obj[0].second.kind == Json::Str;
        if (i == 0 && s.kind == Json::Obj && s.obj.size() == 1 && s.obj[0].first == "Ggml" &&
            s.obj[0].second.kind == Json::Str)
            k.weight = ggml_id(s.obj[0].second.str);
        else if (i == 0 && plain && (s.obj[0].second.str == "F16" || s.obj[0].second.str == "BF16"))
            k.weight = s.obj[0].second.str == "F16" ? SYN_F16 : SYN_BF16;  // gemv/entry.rs:41-47
        else if (!plain_f32)
            k.rest_plain_f32 = false;
    }
    k.layout = u32_of(j.get("layout"), "layout");
    k.variant = u32_of(j.get("variant"), "variant");
    return k;
}

struct Shape {
    uint32_t rows = 0;
    std::vector<uint32_t> dims;
};

Shape parse_shape(const uint8_t* data, size_t len) {
    const Json j = parse(data, len);
    if (j.kind != Json::Obj) fail(SYN_CLASS_INVALID_REQUEST, 0, "ShapeSig: not an object");
    Shape s;
    s.rows = u32_of(j.get("rows"), "rows");
    const Json* dims = j.get("dims");
    if (!dims || dims->kind != Json::Arr) fail(SYN_CLASS_INVALID_REQUEST, 0, "ShapeSig: no dims");
    for (const Json& d : dims->arr) s.dims.push_back(u32_of(&d, "dims"));
    return s;
}

// What one prepared (key, shape) computes.
struct Plan {
    Op op = Op::Other;
    int weight = 0;
    uint32_t rows = 0;
    uint32_t dims[4] = {0, 0, 0, 0};
    uint64_t workspace = 0;  // bytes the executor provides (incl. 256 of alignment slack)
    uint32_t max_block = 0;
    uint32_t accumulate = 1;  // NumericsWire codes: 0 F32, 1 I32ThenF32
    uint32_t act_in = 0;  // NumericsWire codes: 0 none, 2 Q8Block32, 3 Q8K256
    uint32_t layout = 0;  // the weights' LayoutVersion
};

uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// The layout repack gives a dense product's weights of this type (0: they stay in GGUF order).
uint32_t repacked_layout(int weight) {
    return weight == SYN_Q4_K ? SYN_LAYOUT_X8 : weight == SYN_Q8_0 || weight == SYN_Q4_0 ? SYN_LAYOUT_SPLIT : 0;
}

// The plan of a key and shape this provider serves, or false (query answers None).  Gemv and
// MoeGrouped follow the reference's bindings (kernels-cpu/src/gemv/entry.rs:35-66,
// moe/entry.rs:33-56); MoeRoute and MoeCombine their IR signatures
// (crates/graph/src/ir/signature.rs:149,153).
bool plan_of(const Key& k, const Shape& s, Plan& p) {
    if (k.variant != 0 || !k.rest_plain_f32) return false;
    // the repacked layouts are served for the dense products' weights only: 1 (X8) for Q4_K,
    // 2 (SPLIT) for Q8_0 and Q4_0
    if (k.layout != 0 && !(dense(k.op) && k.layout == repacked_layout(k.weight))) return false;
    p.op = k.op;
    p.rows = s.rows;
    p.layout = k.layout;
    switch (k.op) {
    case Op::Gemv:
    case Op::Gemm:
    case Op::Logits:
    case Op::GateUpAct: {
        if (k.weight < 0 || k.n_schemes < 1 || k.n_schemes > 3 || s.dims.size() != 2) return false;
        if (k.op == Op::GateUpAct && !k.silu) return false;  // GELU gating: no reference form yet
        const uint32_t n_out = s.dims[0], k_in = s.dims[1];
        uint64_t ws = 0;
        if (k.op == Op::GateUpAct) {
            if (n_out > (1u << 29) ||
                syn_gate_up_act_workspace_bytes(k.layout, k.weight, s.rows, n_out, k_in, &ws) != SYN_OK)
                return false;
        } else if (k.op == Op::Logits) {
            // room for the normalised rows too (the two-weight binding normalises first)
            if (k_in > 16384 || syn_logits_workspace_bytes(k.layout, k.weight, s.rows, n_out, k_in, &ws) != SYN_OK)
                return false;
        } else if (syn_gemv_layout_workspace_bytes(k.layout, k.weight, s.rows, k_in, &ws) != SYN_OK) {
            return false;
        }
        p.weight = k.weight;
        p.dims[0] = n_out;
        p.dims[1] = k_in;
        p.workspace = round_up(ws, 64) + 256;
        const bool fl = k.weight == SYN_F16 || k.weight == SYN_BF16;
        // F16 / BF16: F32 accumulation of F32 activations (gemv/entry.rs:89-90)
        p.accumulate = fl ? 0 : 1;
        p.max_block = fl ? 0 : k.weight == SYN_Q4_K ? 256 : 32;
        p.act_in = fl ? 0 : k.weight == SYN_Q4_K ? 3 : 2;
        return true;
    }
    case Op::MoeGrouped: {
        // Q4_K or Q8_0 experts (crates/kernels-cpu/src/moe/entry.rs:50-55)
        if ((k.weight != SYN_Q4_K && k.weight != SYN_Q8_0) || k.n_schemes > 3 || s.dims.size() != 4) return false;
        uint64_t ws = 0;
        if (syn_moe_grouped_workspace_bytes(k.weight, s.dims[0], s.dims[1], s.dims[2], s.dims[3],
                                            s.rows, &ws) != SYN_OK)
            return false;
        p.weight = k.weight;
        for (int i = 0; i < 4; ++i) p.dims[i] = s.dims[i];
        p.workspace = round_up(ws, 64) + 256;
        p.max_block = k.weight == SYN_Q4_K ? 256 : 32;
        p.act_in = k.weight == SYN_Q4_K ? 3 : 2;
        return true;
    }
    case Op::MoeRoute: {
        // dims [n_experts, top_k, hidden] (crates/kernels/src/op/kind.rs:242); the router is F32
        if (!k.softmax || k.weight != -1 || s.dims.size() != 3) return false;
        const uint32_t e = s.dims[0], top_k = s.dims[1], hidden = s.dims[2];
        if (e == 0 || e > 256 || top_k == 0 || top_k > e || top_k > 32 || hidden == 0 ||
            hidden % 32 || hidden > 8192)
            return false;
        for (int i = 0; i < 3; ++i) p.dims[i] = s.dims[i];
        // the softmax rows, staged in the workspace (the op's outputs are ids and weights)
        p.workspace = round_up(4ull * s.rows * e, 64) + 256;
        return true;
    }
    case Op::MoeCombine: {
        // dims [top_k, n_shared, hidden] (crates/kernels/src/op/kind.rs:244)
        if (k.weight != -1 || s.dims.size() != 3) return false;
        const uint32_t top_k = s.dims[0], n_shared = s.dims[1], hidden = s.dims[2];
        if (top_k == 0 || top_k > 64 || n_shared > 8 || hidden == 0) return false;
        for (int i = 0; i < 3; ++i) p.dims[i] = s.dims[i];
        p.workspace = 0;
        return true;
    }
    default:
        return false;
    }
}

std::string caps_json(const Plan& p) {
    // CapsWire (wire.rs:762-771) with NumericsWire (:677-686); kernel_hash and source_key are
    // zero: uncertified, as the reference's own kernels until certification
    std::string zeros = "[";
    for (int i = 0; i < 32; ++i) zeros += i ? ",0" : "0";
    zeros += "]";
    const bool route = p.op == Op::MoeRoute, combine = p.op == Op::MoeCombine;
    char num[256];
    std::snprintf(num, sizeof num,
                  "{\"accumulate\":%u,\"max_block\":%u,\"act_in\":%u,\"group\":0,\"out\":0,"
                  "\"softmax_f32\":%s,\"state_f32\":false}",
                  route || combine ? 0u : p.accumulate, p.max_block, p.act_in, route ? "true" : "false");
    return std::string("{\"workspace\":") + std::to_string(p.workspace) + ",\"est\":null,\"layout\":" +
           std::to_string(p.layout) + ",\"capture_safe\":true,\"deterministic\":true,\"numerics\":" + num +
           ",\"kernel_hash\":" + zeros + ",\"source_key\":" + zeros + "}";
}

// ops(): every key served, as the executor's key catalogue (query still decides per shape).
std::string ops_json() {
    std::string out = "[";
    const char* dense_ops[] = {"\"Gemv\"", "\"Gemm\"", "\"Logits\"", "{\"GateUpAct\":{\"act\":\"Silu\"}}"};
    const char* weights[] = {"{\"Ggml\":\"Q4_K\"}", "{\"Ggml\":\"Q8_0\"}", "{\"Ggml\":\"Q4_0\"}",
                             "{\"Ggml\":\"F16\"}", "{\"Ggml\":\"BF16\"}", "{\"Plain\":\"F16\"}",
                             "{\"Plain\":\"BF16\"}"};
    for (const char* op : dense_ops)
        for (const char* w : weights)
            for (int layout = 0; layout < 3; ++layout) {
                const std::string ws(w);
                if (layout == 1 && ws != "{\"Ggml\":\"Q4_K\"}") continue;
                if (layout == 2 && ws != "{\"Ggml\":\"Q8_0\"}" && ws != "{\"Ggml\":\"Q4_0\"}") continue;
                out += std::string("{\"op\":") + op + ",\"schemes\":[" + w +
                       ",{\"Plain\":\"F32\"},{\"Plain\":\"F32\"}],\"layout\":" + std::to_string(layout) +
                       ",\"variant\":0},";
            }
    out +=
        "{\"op\":\"MoeGrouped\",\"schemes\":[{\"Ggml\":\"Q4_K\"},{\"Plain\":\"F32\"},{\"Plain\":\"F32\"}],\"layout\":0,\"variant\":0},"
        "{\"op\":\"MoeGrouped\",\"schemes\":[{\"Ggml\":\"Q8_0\"},{\"Plain\":\"F32\"},{\"Plain\":\"F32\"}],\"layout\":0,\"variant\":0},"
        "{\"op\":{\"MoeRoute\":{\"norm\":\"Softmax\"}},\"schemes\":[{\"Plain\":\"F32\"},{\"Plain\":\"F32\"}],\"layout\":0,\"variant\":0},"
        "{\"op\":\"MoeCombine\",\"schemes\":[{\"Plain\":\"F32\"}],\"layout\":0,\"variant\":0}"
        "]";
    return out;
}

// ============================================================================================
// Contexts
// ============================================================================================

// alloc's memory kinds (crates/kernels/src/memory.rs:33-40)
constexpr uint32_t KIND_DEVICE = 0, KIND_HOST_MAPPED = 1;

struct Buf {
    void* ptr;
    uint64_t bytes;
    uint32_t kind;
    uint32_t first_page;  // HostMapped: the number of its first doorbell page
    uint32_t numbered;    // HostMapped: how many of its pages carry numbers (0: none)
};

// Doorbell flags (RFC-0040 ...md:545-547 and its 2026-11-07 revision at :594): a HostFlag
// {page, slot} names the 4-byte word `slot` of a 4 KiB page of the tier manager's HostMapped
// buffers.  Their pages are numbered in allocation order on the context, from 0, and a number
// is never reused, as the CUDA provider numbers them (crates/kernels-cuda/src/memory.rs:44-49,
// 544-583): a buffer of n bytes takes ceil(n / 4096) numbers (none for 0 bytes); a buffer whose
// pages would pass number 65535 is still allocated, with no numbers (its words hold no flags),
// and does not advance the count.  A HostMapped buffer is pinned, mapped and coherent host
// memory whose device address is its host address (ROCm's unified addressing, checked at
// alloc).
constexpr uint64_t DOORBELL_PAGE = 4096;
constexpr uint32_t MAX_DOORBELL_PAGES = 1u << 16;
constexpr uint64_t DEFAULT_SPIN_US = 2000000;

struct DoorbellPage {
    uint32_t* addr = nullptr;  // host and device address of the page's first word
    uint64_t bytes = 0;        // bytes of the buffer from this page on (the last page may be short)
    bool live = false;
};

// The context's status page: 4 KiB of pinned host memory the kernels write and the host reads
// with plain loads.  Word 0: 1 + (page << 16 | slot) of the first wait_host past its spin limit.
// Words 16-18: the first refused MoeGrouped launch (1 + slot, id, top_k).
constexpr uint32_t STATUS_BELL = 0, STATUS_MOE = 16;

// A host thread's wake target (RFC-0040 ...md:592-600, HostWaker): kind 0 a futex word at
// `handle` that the waiter sets to 1 before it parks (FUTEX_WAIT on 1), kind 1 an eventfd.
struct WakeTarget {
    uint32_t kind;
    uint64_t handle;
};

// The host-function node's body: clears an armed futex word and wakes its waiters, or adds 1 to
// the eventfd.  No HIP call (it runs on the runtime's callback thread).
void wake_target(void* p) {
    const WakeTarget* w = static_cast<const WakeTarget*>(p);
    if (w->kind == 0) {
        uint32_t* word = reinterpret_cast<uint32_t*>(w->handle);
        if (__atomic_exchange_n(word, 0u, __ATOMIC_ACQ_REL) == 1u)
            (void)syscall(SYS_futex, word, FUTEX_WAKE, INT_MAX, nullptr, nullptr, 0);
    } else {
        const uint64_t one = 1;
        (void)!write((int)w->handle, &one, sizeof one);
    }
}

struct Ctx {
    int device = 0;
    uint32_t* status = nullptr;  // the status page (host and device address)
    std::vector<DoorbellPage> pages;
    uint64_t spin_us = DEFAULT_SPIN_US;
    uint64_t spin_ticks = 0;
    // arm_wake: per stream, the side stream its host-function nodes run on, its fork and join
    // events (reused: a wait takes the event's state when it is enqueued), whether a captured
    // fork is still to be joined (at end_capture); and the wake targets the nodes read, one per
    // (kind, handle) at a stable address
    std::unordered_map<uint64_t, hipStream_t> side;
    std::unordered_map<uint64_t, hipEvent_t> fork_ev, join_ev;
    std::unordered_map<uint64_t, bool> forked;
    std::map<std::pair<uint32_t, uint64_t>, WakeTarget> wakes;
    std::unordered_map<uint64_t, Buf> bufs;
    std::unordered_map<uint64_t, hipStream_t> streams;
    std::unordered_map<uint64_t, hipEvent_t> events;
    std::unordered_map<uint64_t, hipGraphExec_t> graphs;
    std::unordered_map<uint64_t, Plan> plans;
    uint64_t next = 1;
    uint64_t handle() { return next++; }
};

std::atomic<uint64_t> g_next_ctx{1};
thread_local std::unordered_map<uint64_t, Ctx*> t_ctx;

Ctx& ctx_of(uint64_t h) {
    auto it = t_ctx.find(h);
    if (it == t_ctx.end())
        internal("context " + std::to_string(h) +
                 " is not open on this thread: a context is used on the thread that opened it");
    check_hip(hipSetDevice(it->second->device), "hipSetDevice");
    return *it->second;
}

hipStream_t stream_of(Ctx& c, uint64_t s) {
    auto it = c.streams.find(s);
    if (it == c.streams.end()) internal("unknown stream " + std::to_string(s));
    return it->second;
}
hipEvent_t event_of(Ctx& c, uint64_t e) {
    auto it = c.events.find(e);
    if (it == c.events.end()) internal("unknown event " + std::to_string(e));
    return it->second;
}
// The word `flag` (page << 16 | slot) names, refused unless it lies in a live HostMapped page.
uint32_t* flag_word(Ctx& c, uint32_t flag) {
    const uint32_t page = flag >> 16, slot = flag & 0xFFFFu;
    if (page >= c.pages.size() || !c.pages[page].live || (uint64_t)slot * 4 + 4 > DOORBELL_PAGE ||
        (uint64_t)slot * 4 + 4 > c.pages[page].bytes)
        internal("no doorbell flag at page " + std::to_string(page) + " slot " + std::to_string(slot) +
                 " on this device");
    return c.pages[page].addr + slot;
}

// What the device reported since the last check, reported once: a wait past its spin limit as
// Timeout / DoorbellTimeout (RFC-0040 ...md:1361), a refused MoeGrouped as Internal, as the CPU
// provider reports MoeError::ExpertId (crates/kernels-cpu/src/moe.rs:433-441, moe/entry.rs:309).
void check_status(Ctx& c) {
    if (!c.status) return;
    const uint32_t tag = __atomic_exchange_n(c.status + STATUS_BELL, 0u, __ATOMIC_ACQ_REL);
    const uint32_t bad = __atomic_load_n(c.status + STATUS_MOE, __ATOMIC_ACQUIRE);
    std::string moe;
    if (bad) {
        const uint32_t id = __atomic_load_n(c.status + STATUS_MOE + 1, __ATOMIC_ACQUIRE);
        const uint32_t k = __atomic_load_n(c.status + STATUS_MOE + 2, __ATOMIC_ACQUIRE);
        __atomic_store_n(c.status + STATUS_MOE, 0u, __ATOMIC_RELEASE);
        const uint32_t slot = bad - 1;
        moe = "MoeGrouped: row " + std::to_string(k ? slot / k : slot) + " rank " + std::to_string(k ? slot % k : 0) +
              " routes to expert " + std::to_string((int32_t)id) +
              ", which the layer lacks; the launch wrote nothing";
        host_log(1, moe);
    }
    if (tag) {
        const uint32_t f = tag - 1;
        std::string m = "wait_host on the doorbell flag at page " + std::to_string(f >> 16) + " slot " +
                        std::to_string(f & 0xFFFFu) + " passed its spin limit of " + std::to_string(c.spin_us) +
                        " us without the host's reply; the stream ran on past it";
        host_log(1, m);
        if (!moe.empty()) m += "; also " + moe;
        fail(SYN_CLASS_TIMEOUT, SYN_CODE_DOORBELL_TIMEOUT, std::move(m));
    }
    if (!moe.empty()) internal(std::move(moe));
}

// The device address of a slice, checked against its buffer.
uint8_t* addr_of(Ctx& c, const SynSlice& s) {
    auto it = c.bufs.find(s.buffer);
    if (it == c.bufs.end()) internal("unknown buffer " + std::to_string(s.buffer));
    if (s.offset > it->second.bytes || s.bytes > it->second.bytes - s.offset)
        internal("a slice runs past its buffer");
    return static_cast<uint8_t*>(it->second.ptr) + s.offset;
}

// A packed tensor argument: dtype, dims [d0, d1, d2, d3] with row-major element strides
// (crates/kernels/src/op/args.rs:85-96), its slice holding the span.
uint8_t* tensor(Ctx& c, const SynTensorArg& t, uint32_t dtype, uint32_t d0, uint32_t d1, uint32_t d2,
                uint32_t elem, const char* what) {
    const uint32_t want[4] = {d0, d1, d2, 1};
    for (int i = 0; i < 4; ++i)
        if (t.dims[i] != want[i])
            internal(std::string(what) + ": dims [" + std::to_string(t.dims[0]) + "," +
                     std::to_string(t.dims[1]) + "," + std::to_string(t.dims[2]) + "," +
                     std::to_string(t.dims[3]) + "] are not the plan's");
    if (t.dtype != dtype) internal(std::string(what) + ": dtype code " + std::to_string(t.dtype));
    // packed: strides[3] = 1 and each stride the product of the extents inside it
    if (t.strides[3] != 1 || t.strides[2] != 1 || t.strides[1] != d2 || t.strides[0] != d1 * d2)
        internal(std::string(what) + " is not packed");
    const uint64_t need = (uint64_t)d0 * d1 * d2 * elem;
    if (t.buf.bytes < need) internal(std::string(what) + ": the slice is shorter than the tensor");
    return addr_of(c, t.buf);
}

uint8_t* workspace_of(Ctx& c, const SynOpArgs& a, const Plan& p) {
    if (p.workspace == 0) return nullptr;
    if (!a.has_workspace || a.workspace.bytes < p.workspace)
        fail(SYN_CLASS_INTERNAL, SYN_CODE_WORKSPACE_EXCEEDED, "the workspace is smaller than the op's caps");
    uint8_t* w = addr_of(c, a.workspace);
    return reinterpret_cast<uint8_t*>(round_up(reinterpret_cast<uintptr_t>(w), 256));
}

// The step descriptor's rows_active (byte offset 8 of syn_step_desc,
// crates/kernels/include/syntropy/step_desc.h:53-57) as a device address the kernels read at
// run time, so that a captured graph follows the value the host writes before each replay; null
// for an empty step slice, which computes the whole bucket (crates/kernels-cpu/src/launch.rs:
// 320-340 reads it the same way on the host).
const uint32_t* step_rows(Ctx& c, const SynOpArgs& a) {
    if (a.step.bytes == 0) return nullptr;
    if (a.step.bytes < 12)
        internal("a " + std::to_string(a.step.bytes) + "-byte step descriptor has no rows_active");
    return reinterpret_cast<const uint32_t*>(addr_of(c, a.step) + 8);
}

const SynBufferView& weight(const SynOpArgs& a, size_t i, uint64_t need, const char* what) {
    if (i >= a.n_weights || !a.weights) internal(std::string(what) + ": missing weight view");
    const SynBufferView& w = a.weights[i];
    if (w.len < need) internal(std::string(what) + ": the weight view is shorter than the matrix");
    return w;
}

void launch_op(Ctx& c, hipStream_t st, const Plan& p, const SynOpArgs& a) {
    const uint32_t rows = p.rows;
    const uint32_t* active = step_rows(c, a);
    switch (p.op) {
    case Op::Gemv:
    case Op::Gemm:
    case Op::Logits:
    case Op::GateUpAct: {
        const bool gated = p.op == Op::GateUpAct;
        const char* name = gated ? "GateUpAct" : p.op == Op::Gemm ? "Gemm" : p.op == Op::Logits ? "Logits" : "Gemv";
        const uint32_t n_out = p.dims[0], k_in = p.dims[1];
        // Logits also takes the final norm (linear.rs:118-161): weight 1 is its F32 [hidden]
        // weight and constant 0 its F32 eps.  With the head alone it is the product of the
        // already-normalised input (the graph's RmsNorm -> Logits, crates/graph/src/blocks/
        // embed.rs:98-135).
        const bool normed = p.op == Op::Logits && a.n_weights == 2;
        if (normed) {
            if (a.n_inputs != 1 || a.n_outputs != 1 || a.n_statics != 1 || a.statics[0].tag != 0)
                internal("Logits with its norm binds one input, one output, the head, the norm weight and an F32 eps");
        } else if (a.n_inputs != 1 || a.n_outputs != 1 || a.n_weights != 1 || a.n_statics != 0) {
            internal(std::string(name) + " binds one input, one output, one weight and no constants");
        }
        const uint8_t* x = tensor(c, a.inputs[0], 0, rows, k_in, 1, 4, "x");
        uint8_t* y = tensor(c, a.outputs[0], 0, rows, n_out, 1, 4, "y");
        const bool fl = p.weight == SYN_F16 || p.weight == SYN_BF16;
        const int be = fl ? 1 : p.weight == SYN_Q4_K ? 256 : 32;
        const int bb = fl ? 2 : p.weight == SYN_Q4_K ? 144 : p.weight == SYN_Q8_0 ? 34 : 18;
        // GateUpAct's weight stacks the gate rows, then the up rows
        const uint64_t wbytes = (uint64_t)k_in / be * bb * n_out * (gated ? 2 : 1);
        const SynBufferView& w = weight(a, 0, wbytes, name);
        // the view's own length: a repacked view must be the repack of this matrix alone
        // (checked by the entry points), a SOURCE view may run past it
        const uint64_t wlen = w.len;
        uint8_t* ws = workspace_of(c, a, p);
        if (normed) {
            const SynBufferView& g = weight(a, 1, 4ull * k_in, "Logits norm");
            float eps;
            std::memcpy(&eps, &a.statics[0].bits, 4);
            check_syn(syn_logits_rows(p.layout, p.weight, (const void*)w.addr, wlen, n_out, k_in,
                                      (const float*)g.addr, eps, (const float*)x, rows, (float*)y, ws,
                                      p.workspace - 256, st, active),
                      name);
        } else if (gated)
            check_syn(syn_gate_up_act_rows(p.layout, p.weight, (const void*)w.addr, wlen, n_out, k_in,
                                           (const float*)x, rows, (float*)y, ws, p.workspace - 256, st, active),
                      name);
        else
            check_syn(syn_gemv_layout_rows(p.layout, p.weight, (const void*)w.addr, wlen, n_out, k_in,
                                           (const float*)x, rows, (float*)y, ws, p.workspace - 256, st, active),
                      name);
        return;
    }
    case Op::MoeGrouped: {
        const uint32_t e = p.dims[0], top_k = p.dims[1], hidden = p.dims[2], inter = p.dims[3];
        if (a.n_inputs < 2 || a.n_inputs > 3 || a.n_outputs != 1 || a.n_weights != 3)
            internal("MoeGrouped binds x, ids (and an optional site), one output and three weights");
        const uint8_t* x = tensor(c, a.inputs[0], 0, rows, hidden, 1, 4, "MoeGrouped x");
        const uint8_t* ids = tensor(c, a.inputs[1], 7, rows, top_k, 1, 4, "MoeGrouped ids");
        // input 2, the site mask: packed I32 [n_experts, 1], nonzero = computed here
        const uint8_t* site = a.n_inputs == 3 ? tensor(c, a.inputs[2], 7, e, 1, 1, 4, "MoeGrouped site") : nullptr;
        uint8_t* out = tensor(c, a.outputs[0], 0, rows, top_k, hidden, 4, "MoeGrouped out");
        const uint64_t mat = p.weight == SYN_Q4_K ? (uint64_t)inter * (hidden / 256) * 144 * e
                                                  : (uint64_t)inter * (hidden / 32) * 34 * e;
        const SynBufferView& g = weight(a, 0, mat, "MoeGrouped gate");
        const SynBufferView& u = weight(a, 1, mat, "MoeGrouped up");
        const SynBufferView& d = weight(a, 2, mat, "MoeGrouped down");
        uint8_t* ws = workspace_of(c, a, p);
        check_syn(syn_moe_grouped_rows(p.weight, (const void*)g.addr, (const void*)u.addr, (const void*)d.addr,
                                       mat, e, top_k, hidden, inter, (const float*)x, (const int32_t*)ids,
                                       (const int32_t*)site, rows,
                                       (float*)out, ws, p.workspace - 256, nullptr, st, active,
                                       c.status + STATUS_MOE),
                  "MoeGrouped");
        return;
    }
    case Op::MoeRoute: {
        const uint32_t e = p.dims[0], top_k = p.dims[1], hidden = p.dims[2];
        if (a.n_inputs != 1 || a.n_outputs != 2 || a.n_weights != 1 || a.n_statics > 1)
            internal("MoeRoute binds x, two outputs (ids, weights), the router and at most one constant");
        // the node's `renormalize` attribute as an I32 or U32 constant; true without one (the
        // Qwen3-MoE norm_topk_prob)
        int renorm = 1;
        if (a.n_statics == 1) {
            if (a.statics[0].tag != 1 && a.statics[0].tag != 2) internal("MoeRoute: renormalize must be an integer constant");
            renorm = a.statics[0].bits != 0;
        }
        const uint8_t* x = tensor(c, a.inputs[0], 0, rows, hidden, 1, 4, "MoeRoute x");
        uint8_t* ids = tensor(c, a.outputs[0], 7, rows, top_k, 1, 4, "MoeRoute ids");
        uint8_t* w = tensor(c, a.outputs[1], 0, rows, top_k, 1, 4, "MoeRoute weights");
        const SynBufferView& r = weight(a, 0, 4ull * e * hidden, "MoeRoute router");
        uint8_t* ws = workspace_of(c, a, p);
        check_syn(syn_moe_route_rows((const float*)r.addr, (const float*)x, rows, hidden, e, top_k, renorm,
                                     (int32_t*)ids, (float*)w, (float*)ws, st, active),
                  "MoeRoute");
        return;
    }
    case Op::MoeCombine: {
        // inputs [per_expert F32 [rows, top_k, hidden], weights F32 [rows, top_k], then each shared
        // expert's output F32 [rows, hidden]] (crates/graph/src/ir/signature.rs:153,
        // crates/graph/src/blocks/ffn.rs:189-200); slots added in rank order, then the shared
        // outputs
        const uint32_t top_k = p.dims[0], n_shared = p.dims[1], hidden = p.dims[2];
        if (a.n_inputs != 2 + (size_t)n_shared || a.n_outputs != 1 || a.n_weights != 0 || a.n_statics != 0)
            internal("MoeCombine binds the per-expert outputs, their weights, n_shared shared outputs and one output");
        const uint8_t* per = tensor(c, a.inputs[0], 0, rows, top_k, hidden, 4, "MoeCombine outputs");
        const uint8_t* w = tensor(c, a.inputs[1], 0, rows, top_k, 1, 4, "MoeCombine weights");
        const float* shared[8] = {};
        for (uint32_t i = 0; i < n_shared; ++i)
            shared[i] = (const float*)tensor(c, a.inputs[2 + i], 0, rows, hidden, 1, 4, "MoeCombine shared output");
        uint8_t* y = tensor(c, a.outputs[0], 0, rows, hidden, 1, 4, "MoeCombine y");
        check_syn(syn_moe_combine_ranked_rows((const float*)per, (const float*)w, n_shared, shared, rows, top_k,
                                              hidden, (float*)y, st, active),
                  "MoeCombine");
        return;
    }
    default:
        internal("a prepared op of no kind");
    }
}

// ============================================================================================
// The table's entries
// ============================================================================================

SynStatus e_build(void*, SynOutBuf* out) {
    return call("build", false, [&] {
        int rt = 0;
        (void)hipRuntimeGetVersion(&rt);
        put(out, "{\"version\":1,\"module\":null,\"toolchain\":[[\"hip\",\"" + std::to_string(rt) +
                     "\"],[\"target\",\"gfx950\"]],\"driver\":null}");
    });
}

SynStatus e_enumerate(void*, SynOutBuf* out) {
    return call("enumerate", false, [&] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        std::string s = "[";
        for (int i = 0; i < n; ++i) {
            hipDeviceProp_t prop{};
            check_hip(hipGetDeviceProperties(&prop, i), "hipGetDeviceProperties");
            size_t free_b = 0, total_b = 0;
            check_hip(hipSetDevice(i), "hipSetDevice");
            check_hip(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
            char rec[768];
            std::snprintf(rec, sizeof rec,
                          "%s{\"local\":%d,\"uuid\":null,\"pci\":{\"domain\":%d,\"bus\":%d,\"device\":%d,\"function\":0},"
                          "\"kind\":\"DiscreteGpu\",\"name\":\"%s\",\"class\":{\"Hip\":{\"gfx\":%d}},\"features\":0,"
                          "\"memory\":{\"total\":%zu,\"free\":%zu,\"budget\":null,\"host_visible_device_local\":null,"
                          "\"max_alloc\":%zu,\"unified\":false},\"numa\":null}",
                          i ? "," : "", i, prop.pciDomainID, prop.pciBusID, prop.pciDeviceID, "AMD Instinct MI355X",
                          0x950, total_b, free_b, total_b);
            s += rec;
        }
        put(out, s + "]");
    });
}

SynStatus e_open(void*, const SynDeviceId* dev, const SynOpenOptions* opts, uint64_t* ctx) {
    return call("open", false, [&] {
        if (!dev || !ctx) internal("open: null argument");
        (void)opts;  // doorbell pages are the tier manager's HostMapped buffers (RFC-0040 ...md:594)
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0) fail(SYN_CLASS_DEVICE, 0, "open: no HIP device");
        if ((int)dev->ordinal >= n) fail(SYN_CLASS_INVALID_REQUEST, 0, "open: no device " + std::to_string(dev->ordinal));
        check_hip(hipSetDevice((int)dev->ordinal), "hipSetDevice");
        // the bound of one wait_host: the core's kernels.spin_kernel_max_us (RFC-0040 ...md:1342),
        // 2 s when the core sets none
        uint64_t spin_us = DEFAULT_SPIN_US;
        if (const char* v = host_config("kernels.spin_kernel_max_us")) {
            char* end = nullptr;
            const unsigned long long u = std::strtoull(v, &end, 10);
            if (end == v || *end || u == 0 || u > 600000000ull)
                fail(SYN_CLASS_INVALID_REQUEST, 0,
                     std::string("open: kernels.spin_kernel_max_us must be 1..600000000, not '") + v + "'");
            spin_us = u;
        }
        int khz = 0;
        check_hip(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, (int)dev->ordinal),
                  "hipDeviceGetAttribute(WallClockRate)");
        if (khz <= 0) fail(SYN_CLASS_DEVICE, 0, "open: the device reports no wall-clock rate");
        // the status page: the one allocation outside the tier manager's requests, 4 KiB per
        // context, for the words the kernels report through
        void* st = nullptr;
        check_hip(hipHostMalloc(&st, DOORBELL_PAGE, hipHostMallocMapped | hipHostMallocCoherent),
                  "hipHostMalloc(status page)");
        std::memset(st, 0, DOORBELL_PAGE);
        void* st_dev = nullptr;
        const hipError_t r = hipHostGetDevicePointer(&st_dev, st, 0);
        if (r != hipSuccess || st_dev != st) {
            (void)hipHostFree(st);
            check_hip(r == hipSuccess ? hipErrorInvalidValue : r, "hipHostGetDevicePointer(status page)");
        }
        Ctx* c = new Ctx();
        c->device = (int)dev->ordinal;
        c->status = static_cast<uint32_t*>(st);
        c->spin_us = spin_us;
        c->spin_ticks = spin_us * (uint64_t)khz / 1000u;
        const uint64_t h = g_next_ctx.fetch_add(1);
        t_ctx[h] = c;
        *ctx = h;
    });
}

void free_buf(const Buf& b) {
    if (b.kind == KIND_HOST_MAPPED) (void)hipHostFree(b.ptr);
    else (void)hipFree(b.ptr);
}

SynStatus e_close_ctx(void*, uint64_t ctx) {
    return call("close_ctx", true, [&] {
        auto it = t_ctx.find(ctx);
        if (it == t_ctx.end())
            internal("context " + std::to_string(ctx) + " is not open on this thread, so it was not closed");
        Ctx* c = it->second;
        (void)hipSetDevice(c->device);
        for (auto& g : c->graphs) (void)hipGraphExecDestroy(g.second);
        for (auto& e : c->events) (void)hipEventDestroy(e.second);
        for (auto& s : c->side) {
            (void)hipStreamSynchronize(s.second);  // pending wakes run before their targets go
            (void)hipStreamDestroy(s.second);
        }
        for (auto& e : c->fork_ev) (void)hipEventDestroy(e.second);
        for (auto& e : c->join_ev) (void)hipEventDestroy(e.second);
        for (auto& s : c->streams) (void)hipStreamDestroy(s.second);
        for (auto& b : c->bufs) free_buf(b.second);
        if (c->status) (void)hipHostFree(c->status);
        delete c;
        t_ctx.erase(it);
    });
}

SynStatus e_memory_info(void*, uint64_t ctx, SynMemoryInfo* out) {
    return call("memory_info", false, [&] {
        ctx_of(ctx);
        size_t free_b = 0, total_b = 0;
        check_hip(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
        SynMemoryInfo m{};
        m.total = total_b;
        m.free = free_b;
        m.max_alloc = total_b;
        *out = m;
    });
}

SynStatus e_ops(void*, SynOutBuf* out) {
    return call("ops", false, [&] {
        static const std::string ops = ops_json();
        put(out, ops);
    });
}

SynStatus e_query(void*, uint64_t ctx, const uint8_t* op, size_t op_len, const uint8_t* shape,
                  size_t shape_len, SynOutBuf* out) {
    return call("query", false, [&] {
        ctx_of(ctx);
        const Key k = parse_key(op, op_len);
        const Shape s = parse_shape(shape, shape_len);
        Plan p;
        put(out, plan_of(k, s, p) ? caps_json(p) : std::string());
    });
}

// alloc (RFC-0040 ...md §5.1): Device as hipMalloc; HostMapped as pinned, mapped, coherent host
// pages (hipHostMalloc), zeroed, whose 4 KiB pages become the next doorbell pages.
SynStatus e_alloc(void*, uint64_t ctx, const SynAllocRequest* req, SynBuffer* out) {
    return call("alloc", false, [&] {
        Ctx& c = ctx_of(ctx);
        if (!req || !out) internal("alloc: null argument");
        if (req->reserve_only || (req->kind != KIND_DEVICE && req->kind != KIND_HOST_MAPPED))
            unsupported("alloc: Device and HostMapped memory are served, without reservations");
        if (req->align > 256 && (req->align & (req->align - 1))) internal("alloc: alignment is not a power of two");
        if (req->kind == KIND_HOST_MAPPED && req->align > DOORBELL_PAGE)
            unsupported("alloc: HostMapped memory is aligned to 4 KiB pages");
        void* p = nullptr;
        uint32_t first_page = 0, numbered = 0;
        if (req->kind == KIND_DEVICE) {
            if (hipMalloc(&p, req->bytes ? req->bytes : 1) != hipSuccess)
                fail(SYN_CLASS_CAPACITY, SYN_CODE_ALLOC_FAILED, "alloc: " + std::to_string(req->bytes) + " bytes");
        } else {
            const uint64_t pages = (req->bytes + DOORBELL_PAGE - 1) / DOORBELL_PAGE;
            if (hipHostMalloc(&p, (pages ? pages : 1) * DOORBELL_PAGE, hipHostMallocMapped | hipHostMallocCoherent) !=
                hipSuccess)
                fail(SYN_CLASS_CAPACITY, SYN_CODE_ALLOC_FAILED,
                     "alloc: " + std::to_string(req->bytes) + " bytes of host-mapped memory");
            void* d = nullptr;
            if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess || d != p) {
                (void)hipHostFree(p);
                fail(SYN_CLASS_DEVICE, 0, "alloc: host-mapped memory whose device address is not its host address");
            }
            std::memset(p, 0, (pages ? pages : 1) * DOORBELL_PAGE);
            first_page = (uint32_t)c.pages.size();
            if (first_page + pages <= MAX_DOORBELL_PAGES) {  // else the buffer carries no numbers
                numbered = (uint32_t)pages;
                for (uint64_t i = 0; i < pages; ++i) {
                    DoorbellPage pg;
                    pg.addr = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + i * DOORBELL_PAGE);
                    pg.bytes = req->bytes - i * DOORBELL_PAGE;
                    pg.live = true;
                    c.pages.push_back(pg);
                }
            }
        }
        const uint64_t h = c.handle();
        c.bufs[h] = Buf{p, req->bytes, req->kind, first_page, numbered};
        SynBuffer b{};
        b.addr = reinterpret_cast<uint64_t>(p);
        b.bytes = req->bytes;
        b.handle = h;
        b.kind = req->kind;
        *out = b;
    });
}

SynStatus e_free(void*, uint64_t ctx, const SynBuffer* buf) {
    return call("free", true, [&] {
        Ctx& c = ctx_of(ctx);
        if (!buf) internal("free: null buffer");
        auto it = c.bufs.find(buf->handle);
        if (it == c.bufs.end()) internal("free: unknown buffer " + std::to_string(buf->handle));
        const Buf b = it->second;
        if (b.kind == KIND_HOST_MAPPED) {  // its page numbers retire, never renaming another flag
            for (uint32_t i = 0; i < b.numbered; ++i) c.pages[b.first_page + i].live = false;
            check_hip(hipHostFree(b.ptr), "hipHostFree");
        } else {
            check_hip(hipFree(b.ptr), "hipFree");
        }
        c.bufs.erase(it);
    });
}

#define SYN_UNSERVED(name, ...)                                                   \
    SynStatus e_##name(__VA_ARGS__) {                                             \
        return call(#name, false, [&] { unsupported("`" #name "` is not served by the hip provider"); }); \
    }
SYN_UNSERVED(map_segment, void*, uint64_t, const SynBuffer*, uint64_t, uint64_t, SynSegment*)
SYN_UNSERVED(unmap_segment, void*, uint64_t, const SynSegment*)
SYN_UNSERVED(register_host, void*, uint64_t, SynHostRegion, SynRegistration*)
SYN_UNSERVED(host_registrar, void*, uint64_t, SynRegistrarVtbl*)
SYN_UNSERVED(import, void*, uint64_t, SynHostRegion, SynBuffer*)
#undef SYN_UNSERVED

SynStatus e_set_resident(void*, uint64_t ctx, const SynBuffer*, size_t, uint32_t) {
    // device memory is always resident
    return call("set_resident", false, [&] { ctx_of(ctx); });
}

// The dense products' Q4_K weights are repacked to layout 1 (X8: each run of eight super-blocks
// stored chunk-major), their Q8_0 and Q4_0 weights to layout 2 (SPLIT: every block's codes, then
// every block's F16 scale).  Both are permutations of the bytes, so the same length.  Every other
// op's weights keep their GGUF layout (LayoutVersion SOURCE, `present` 0).
uint32_t repack_target(const uint8_t* op, size_t op_len, int* weight) {
    const Key k = parse_key(op, op_len);
    *weight = k.weight;
    return dense(k.op) && k.layout == 0 ? repacked_layout(k.weight) : 0;
}
SynStatus e_repack(void*, const uint8_t* op, size_t op_len, const uint8_t* src, size_t src_len, uint8_t* dst,
                   size_t dst_len, uint32_t* present, uint32_t* layout) {
    return call("repack", false, [&] {
        if (!present || !layout) internal("repack: null output");
        *present = 0;
        *layout = 0;
        int weight = 0;
        const uint32_t to = repack_target(op, op_len, &weight);
        if (to == 0) return;
        if (dst_len < src_len) fail(SYN_CLASS_INVALID_REQUEST, 0, "repack: the destination is shorter than the source");
        if (to == SYN_LAYOUT_X8) {
            if (src_len % 144) fail(SYN_CLASS_INVALID_REQUEST, 0, "repack: the bytes are not whole Q4_K super-blocks");
            check_syn(syn_q4k_repack_host(SYN_LAYOUT_X8, src, dst, src_len, 0), "repack");
        } else {
            if (src_len % (weight == SYN_Q8_0 ? 34 : 18))
                fail(SYN_CLASS_INVALID_REQUEST, 0, "repack: the bytes are not whole 32-value blocks");
            check_syn(syn_split_repack_host(SYN_LAYOUT_SPLIT, weight, src, dst, src_len, 0), "repack");
        }
        *present = 1;
        *layout = to;
    });
}
SynStatus e_repacked_len(void*, const uint8_t* op, size_t op_len, uint64_t src, uint32_t* present, uint64_t* out) {
    return call("repacked_len", false, [&] {
        if (!present || !out) internal("repacked_len: null output");
        int weight = 0;
        *present = repack_target(op, op_len, &weight) != 0 ? 1 : 0;
        *out = *present ? src : 0;
    });
}

SynStatus e_stream(void*, uint64_t ctx, uint32_t prio, uint64_t* out) {
    return call("stream", false, [&] {
        Ctx& c = ctx_of(ctx);
        if (prio > 4) internal("stream: unknown priority code " + std::to_string(prio));
        // every stream at the default priority: the priority code only names the stream's role
        hipStream_t s = nullptr;
        check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        const uint64_t h = c.handle();
        c.streams[h] = s;
        *out = h;
    });
}

SynStatus e_event(void*, uint64_t ctx, uint64_t* out) {
    return call("event", false, [&] {
        Ctx& c = ctx_of(ctx);
        hipEvent_t e = nullptr;
        check_hip(hipEventCreate(&e), "hipEventCreate");
        const uint64_t h = c.handle();
        c.events[h] = e;
        *out = h;
    });
}

SynStatus e_record(void*, uint64_t ctx, uint64_t s, uint64_t e) {
    return call("record", false, [&] {
        Ctx& c = ctx_of(ctx);
        check_hip(hipEventRecord(event_of(c, e), stream_of(c, s)), "hipEventRecord");
    });
}

SynStatus e_wait(void*, uint64_t ctx, uint64_t s, uint64_t e) {
    return call("wait", false, [&] {
        Ctx& c = ctx_of(ctx);
        check_hip(hipStreamWaitEvent(stream_of(c, s), event_of(c, e), 0), "hipStreamWaitEvent");
    });
}

// signal_host: a one-lane store kernel writes `value` to the flag when the stream reaches it
// (provider.rs:346-356; RFC-0040 ...md:549-553, the store kernel).
SynStatus e_signal_host(void*, uint64_t ctx, uint64_t s, uint32_t flag, uint32_t value) {
    return call("signal_host", false, [&] {
        Ctx& c = ctx_of(ctx);
        hipStream_t st = stream_of(c, s);
        syn::launch_bell_signal(flag_word(c, flag), value, st);
        check_hip(hipGetLastError(), "signal_host");
    });
}

// wait_host: a one-wave kernel holds the stream until the flag compares Eq (cmp 0) or Geq (1)
// with `value`, then writes `reset` when has_reset is 1 (provider.rs:357-377).  The wait gives up
// after the spin limit; synchronize then reports a Timeout (RFC-0040 ...md:579-584).
SynStatus e_wait_host(void*, uint64_t ctx, uint64_t s, uint32_t flag, uint32_t value, uint32_t cmp,
                      uint32_t has_reset, uint32_t reset) {
    return call("wait_host", false, [&] {
        Ctx& c = ctx_of(ctx);
        if (cmp > 1) internal("wait_host: comparison code " + std::to_string(cmp) + " (0 Eq, 1 Geq)");
        if (has_reset > 1) internal("wait_host: has_reset must be 0 or 1");
        hipStream_t st = stream_of(c, s);
        syn::launch_bell_wait(flag_word(c, flag), value, (int)cmp, (int)has_reset, reset, c.spin_ticks,
                              c.status + STATUS_BELL, flag + 1u, st);
        check_hip(hipGetLastError(), "wait_host");
    });
}

// arm_wake (provider.rs:378-384; RFC-0040 ...md:590-600, the HIP row): a host-function node on
// a side branch forked from `s` at this point, so the wake follows the work enqueued so far
// (normally a doorbell write) and `s` never waits for it; a captured branch is joined back at
// end_capture, the step's end.  Kinds: 0 Futex (handle: the word's address), 1 EventFd
// (handle: the descriptor); WinEvent and TimelineValue are not served.
SynStatus e_arm_wake(void*, uint64_t ctx, uint64_t s, uint32_t kind, uint64_t handle) {
    return call("arm_wake", false, [&] {
        if (kind > 1) unsupported("arm_wake: wake kind " + std::to_string(kind) + " (Futex 0 and EventFd 1 only)");
        Ctx& c = ctx_of(ctx);
        if (kind == 0 && (handle == 0 || handle % 4)) internal("arm_wake: a futex word must be a 4-byte aligned address");
        if (kind == 1 && handle > (uint64_t)INT_MAX) internal("arm_wake: not a file descriptor");
        hipStream_t st = stream_of(c, s);
        hipStream_t& side = c.side[s];
        if (!side) check_hip(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "hipStreamCreate(arm_wake)");
        hipEvent_t& ev = c.fork_ev[s];
        if (!ev) check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate(arm_wake)");
        WakeTarget& target = c.wakes.emplace(std::make_pair(kind, handle), WakeTarget{kind, handle}).first->second;
        check_hip(hipEventRecord(ev, st), "hipEventRecord(arm_wake)");
        check_hip(hipStreamWaitEvent(side, ev, 0), "hipStreamWaitEvent(arm_wake)");
        check_hip(hipLaunchHostFunc(side, wake_target, &target), "hipLaunchHostFunc(arm_wake)");
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        check_hip(hipStreamIsCapturing(st, &cap), "hipStreamIsCapturing");
        if (cap == hipStreamCaptureStatusActive) c.forked[s] = true;  // joined at end_capture
    });
}

SynStatus e_poll(void*, uint64_t ctx, uint64_t e, uint32_t* done) {
    return call("poll", false, [&] {
        Ctx& c = ctx_of(ctx);
        const hipError_t r = hipEventQuery(event_of(c, e));
        if (r == hipSuccess) *done = 1;
        else if (r == hipErrorNotReady) *done = 0;
        else check_hip(r, "hipEventQuery");
        if (*done) check_status(c);
    });
}

SynStatus e_elapsed(void*, uint64_t ctx, uint64_t start, uint64_t end, uint32_t* present, uint64_t* nanos) {
    return call("elapsed", false, [&] {
        Ctx& c = ctx_of(ctx);
        float ms = 0.0f;
        const hipError_t r = hipEventElapsedTime(&ms, event_of(c, start), event_of(c, end));
        if (r == hipSuccess) {
            *present = 1;
            *nanos = (uint64_t)((double)ms * 1e6);
        } else {
            *present = 0;
            *nanos = 0;
        }
    });
}

SynStatus e_synchronize(void*, uint64_t ctx, uint64_t s) {
    return call("synchronize", false, [&] {
        Ctx& c = ctx_of(ctx);
        check_hip(hipStreamSynchronize(stream_of(c, s)), "hipStreamSynchronize");
        check_status(c);
    });
}

void copy_one(Ctx& c, hipStream_t st, const SynSlice& src, const SynSlice& dst) {
    if (src.bytes != dst.bytes) internal("copy: the slices differ in length");
    // device and host-mapped buffers alike (one address space)
    check_hip(hipMemcpyAsync(addr_of(c, dst), addr_of(c, src), src.bytes, hipMemcpyDefault, st), "hipMemcpyAsync");
}

SynStatus e_copy(void*, uint64_t ctx, uint64_t s, const SynSlice* src, const SynSlice* dst) {
    return call("copy", false, [&] {
        Ctx& c = ctx_of(ctx);
        copy_one(c, stream_of(c, s), *src, *dst);
    });
}

SynStatus e_copy_batch(void*, uint64_t ctx, uint64_t s, const SynSlicePair* pairs, size_t n) {
    return call("copy_batch", false, [&] {
        Ctx& c = ctx_of(ctx);
        hipStream_t st = stream_of(c, s);
        for (size_t i = 0; i < n; ++i) copy_one(c, st, pairs[i].src, pairs[i].dst);
    });
}

SynStatus e_prepare(void*, uint64_t ctx, const uint8_t* op, size_t op_len, const uint8_t* shape,
                    size_t shape_len, SynPreparedOp* out) {
    return call("prepare", false, [&] {
        Ctx& c = ctx_of(ctx);
        const Key k = parse_key(op, op_len);
        const Shape s = parse_shape(shape, shape_len);
        Plan p;
        if (!plan_of(k, s, p)) unsupported("prepare: an op or shape the hip provider does not serve");
        const uint64_t h = c.handle();
        c.plans[h] = p;
        SynPreparedOp r;
        r.workspace = p.workspace;
        r.handle = h;
        *out = r;
    });
}

SynStatus e_launch(void*, uint64_t ctx, uint64_t s, const SynPreparedOp* op, const SynOpArgs* args) {
    return call("launch", false, [&] {
        Ctx& c = ctx_of(ctx);
        if (!op || !args) internal("launch: null argument");
        auto it = c.plans.find(op->handle);
        if (it == c.plans.end()) internal("launch: unknown prepared op " + std::to_string(op->handle));
        launch_op(c, stream_of(c, s), it->second, *args);
    });
}

SynStatus e_begin_capture(void*, uint64_t ctx, uint64_t s) {
    return call("begin_capture", false, [&] {
        Ctx& c = ctx_of(ctx);
        check_hip(hipStreamBeginCapture(stream_of(c, s), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    });
}

SynStatus e_end_capture(void*, uint64_t ctx, uint64_t s, uint64_t* out) {
    return call("end_capture", false, [&] {
        Ctx& c = ctx_of(ctx);
        if (c.forked[s]) {  // join the wakes' branch back: the captured step ends after them
            hipEvent_t& ev = c.join_ev[s];
            if (!ev) check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate(join)");
            check_hip(hipEventRecord(ev, c.side[s]), "hipEventRecord(join)");
            check_hip(hipStreamWaitEvent(stream_of(c, s), ev, 0), "hipStreamWaitEvent(join)");
            c.forked[s] = false;
        }
        hipGraph_t g = nullptr;
        check_hip(hipStreamEndCapture(stream_of(c, s), &g), "hipStreamEndCapture");
        hipGraphExec_t ex = nullptr;
        const hipError_t r = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        check_hip(r, "hipGraphInstantiate");
        const uint64_t h = c.handle();
        c.graphs[h] = ex;
        *out = h;
    });
}

SynStatus e_replay(void*, uint64_t ctx, uint64_t s, uint64_t g) {
    return call("replay", false, [&] {
        Ctx& c = ctx_of(ctx);
        auto it = c.graphs.find(g);
        if (it == c.graphs.end()) internal("replay: unknown graph " + std::to_string(g));
        check_hip(hipGraphLaunch(it->second, stream_of(c, s)), "hipGraphLaunch");
    });
}

SynStatus e_health(void*, uint64_t ctx, SynHealth* out) {
    return call("health", true, [&] {
        (void)ctx;
        SynHealth h{};
        const uint16_t sticky = g_sticky.load(std::memory_order_acquire);
        if (sticky) {  // Sticky, in the Kernels domain, with the code that made it so
            h.kind = 3;
            h.domain = SYN_DOMAIN_KERNELS;
            h.detail = sticky;
        }
        *out = h;
    });
}

SynStatus e_last_error(void*, uint64_t, uint8_t* buf, size_t cap, size_t* len) {
    // never refused: it reports why the last call failed
    const std::string& m = t_message;
    if (len) *len = m.size();
    if (buf) std::memcpy(buf, m.data(), m.size() < cap ? m.size() : cap);
    return OK;
}

SynStatus e_shutdown() { return OK; }

SynHeader header(uint32_t size) {
    SynHeader h{};
    std::memcpy(h.magic, SYN_PROVIDER_MAGIC, 8);
    h.abi_major = SYN_ABI_MAJOR;
    h.abi_minor = SYN_ABI_MINOR;
    // build id: zero, so the core accepts the module under kernels.dev_modules only
    h.struct_size = size;
    return h;
}

SynProviderVtbl make_vtbl() {
    SynProviderVtbl v{};
    v.struct_size = sizeof(SynProviderVtbl);
    v.id = "hip";
    v.backend = SYN_BACKEND_HIP;
    v.domain = SYN_MEMDOMAIN_HIP;
    v.build = e_build;
    v.enumerate = e_enumerate;
    v.open = e_open;
    v.close_ctx = e_close_ctx;
    v.memory_info = e_memory_info;
    v.ops = e_ops;
    v.query = e_query;
    v.alloc = e_alloc;
    v.free = e_free;
    v.map_segment = e_map_segment;
    v.unmap_segment = e_unmap_segment;
    v.register_host = e_register_host;
    v.host_registrar = e_host_registrar;
    v.import = e_import;
    v.set_resident = e_set_resident;
    v.repack = e_repack;
    v.repacked_len = e_repacked_len;
    v.stream = e_stream;
    v.event = e_event;
    v.record = e_record;
    v.wait = e_wait;
    v.signal_host = e_signal_host;
    v.wait_host = e_wait_host;
    v.arm_wake = e_arm_wake;
    v.poll = e_poll;
    v.elapsed = e_elapsed;
    v.synchronize = e_synchronize;
    v.copy = e_copy;
    v.copy_batch = e_copy_batch;
    v.prepare = e_prepare;
    v.launch = e_launch;
    v.begin_capture = e_begin_capture;
    v.end_capture = e_end_capture;
    v.replay = e_replay;
    v.health = e_health;
    v.last_error = e_last_error;
    v.slf = nullptr;
    v.health_size = sizeof(SynHealth);
    return v;
}

const SynProviderVtbl g_vtbl = make_vtbl();
const SynModule g_module = {header(sizeof(SynModule)), 1, &g_vtbl, e_shutdown};

}  // namespace

SYN_PROVIDER_EXPORT const SynModule* syntropy_provider_entry_v1(const SynHostApi* host) {
    // the module checks the host's magic, major and size (RFC-0040 §10.4; module.rs:26-40)
    if (!host || std::memcmp(host->h.magic, SYN_PROVIDER_MAGIC, 8) != 0 ||
        host->h.abi_major != SYN_ABI_MAJOR || host->h.struct_size < sizeof(SynHostApi))
        return nullptr;
    // the services are kept for the module's life; the fault-injection keys are read now
    std::call_once(g_host_once, [&] {
        g_host.api = *host;
        g_host.present = true;
        if (const char* v = host_config("fixture.panic_in")) g_host.panic_in = v;
        if (const char* v = host_config("fixture.device_fault_in")) g_host.device_fault_in = v;
    });
    return &g_module;
}
