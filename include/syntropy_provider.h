/* The provider-library boundary: the one symbol a kernel module exports and the tables it
 * returns, laid out field for field as the reference core expects them
 * (crates/kernels/src/abi/types.rs, mod.rs, status.rs).  Field order is the ABI; a minor
 * version only appends.  Each side frees what it allocated; variable-size results go through a
 * caller buffer (SynOutBuf); handles are opaque 64-bit values.
 *
 * libsyntropy_provider.so exports exactly syntropy_provider_entry_v1, under the version node
 * SYNTROPY_PROVIDER_1 (the reference's ci/link/provider.map), and is linked -Bsymbolic.
 *
 * Doorbell flags: signal_host and wait_host take `flag` = page << 16 | slot, naming the 4-byte
 * word `slot` of a 4 KiB page of the HostMapped buffers (alloc kind 1) of the context.  Their
 * pages are numbered in allocation order from 0 and never reused (RFC-0040 4.2, revised
 * 2026-11-07).  A HostMapped buffer's `addr` is both its device and its host address. */
#ifndef SYNTROPY_PROVIDER_H
#define SYNTROPY_PROVIDER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SYN_PROVIDER_MAGIC "SYNPROV1"
#define SYN_ABI_MAJOR 1u /* crates/kernels/src/abi/mod.rs: ABI_MAJOR */
#define SYN_ABI_MINOR 0u /* mod.rs: ABI_MINOR */
#define SYN_DOMAIN_KERNELS 1u /* mod.rs: DOMAIN_KERNELS */
#define SYN_BACKEND_HIP 2u /* wire.rs: backend_code(Backend::Hip) */
#define SYN_MEMDOMAIN_HIP 2u /* wire.rs: domain_code(MemoryDomain::Hip) */

/* Error classes (status.rs: class_code) and the Kernels domain's codes (RFC-0040 §13, the
 * reference's crates/core/src/error/codes.rs: kernels). */
enum {
    SYN_CLASS_OK = 0,
    SYN_CLASS_INVALID_REQUEST = 1,
    SYN_CLASS_UNSUPPORTED = 2,
    SYN_CLASS_CAPACITY = 3,
    SYN_CLASS_DEVICE = 6,
    SYN_CLASS_TIMEOUT = 10,
    SYN_CLASS_INTERNAL = 13
};
enum {
    SYN_CODE_OP_UNSUPPORTED = 1,
    SYN_CODE_DEVICE_STICKY = 8,
    SYN_CODE_ALLOC_FAILED = 9,
    SYN_CODE_DOORBELL_TIMEOUT = 11,
    SYN_CODE_WORKSPACE_EXCEEDED = 14,
    SYN_CODE_PROVIDER_PANICKED = 16
};

/* types.rs:16-27 */
typedef struct SynHeader {
    uint8_t magic[8];
    uint32_t abi_major;
    uint32_t abi_minor;
    uint8_t build_id[32];
    uint32_t struct_size;
} SynHeader;

/* status.rs: SynStatus{class, domain, code, retry} (`cls` is the reference's `class`) */
typedef struct SynStatus {
    uint32_t cls;
    uint32_t domain;
    uint16_t code;
    uint8_t retry;
} SynStatus;

/* types.rs:47-58 */
typedef struct SynHostApi {
    SynHeader h;
    void (*log)(uint8_t level, const char* target, const char* msg, size_t len);
    void (*metric)(uint32_t id, uint64_t value);
    const char* (*config)(const char* key);
} SynHostApi;

/* types.rs:62-68 */
typedef struct SynDeviceId {
    uint8_t node[32];
    uint32_t ordinal;
} SynDeviceId;

/* types.rs:72-85 */
typedef struct SynOpenOptions {
    uint8_t streams[4];
    uint32_t doorbell_slots;
    uint8_t capture;
    uint8_t deterministic;
    uint8_t power;
    uint8_t reserved;
} SynOpenOptions;

/* types.rs:90-104 */
typedef struct SynMemoryInfo {
    uint64_t total;
    uint64_t free;
    uint64_t budget;
    uint64_t host_visible;
    uint64_t max_alloc;
    uint32_t flags;
    uint32_t reserved;
} SynMemoryInfo;

/* types.rs:108-117 */
typedef struct SynAllocRequest {
    uint64_t bytes;
    uint64_t align;
    uint32_t kind;
    uint32_t reserve_only;
} SynAllocRequest;

/* types.rs:121-132 */
typedef struct SynBuffer {
    uint64_t addr;
    uint64_t bytes;
    uint64_t handle;
    uint32_t kind;
    uint32_t reserved;
} SynBuffer;

/* types.rs:142-149: `buffer` is a handle from alloc */
typedef struct SynSlice {
    uint64_t buffer;
    uint64_t offset;
    uint64_t bytes;
} SynSlice;

typedef struct SynSlicePair {
    SynSlice src;
    SynSlice dst;
} SynSlicePair;

typedef struct SynSegment {
    uint64_t reservation;
    uint64_t offset;
    uint64_t bytes;
    uint64_t handle;
} SynSegment;

typedef struct SynHostRegion {
    uint64_t addr;
    uint64_t len;
} SynHostRegion;

typedef struct SynRegistration {
    SynHostRegion region;
    uint64_t handle;
} SynRegistration;

/* types.rs: SynHealth (12 bytes: health_size) */
typedef struct SynHealth {
    uint32_t kind;
    uint32_t domain;
    uint32_t detail;
} SynHealth;

typedef struct SynPreparedOp {
    uint64_t workspace;
    uint64_t handle;
} SynPreparedOp;

/* types.rs:224-235: dims and strides in elements; dtype = index in DType::ALL (F32 0, F16 1,
 * BF16 2, I8 5, U8 6, I32 7) */
typedef struct SynTensorArg {
    SynSlice buf;
    uint32_t dtype;
    uint32_t reserved;
    uint32_t dims[4];
    uint32_t strides[4];
} SynTensorArg;

/* a weight view: `addr` is the device address of `len` bytes */
typedef struct SynBufferView {
    uint32_t kind;
    uint32_t ordinal;
    uint8_t node[32];
    uint64_t addr;
    uint64_t len;
} SynBufferView;

typedef struct SynScalar {
    uint32_t tag;
    uint32_t bits;
} SynScalar;

/* types.rs:267-292 */
typedef struct SynOpArgs {
    uint32_t struct_size;
    uint32_t has_workspace;
    const SynTensorArg* inputs;
    size_t n_inputs;
    const SynTensorArg* outputs;
    size_t n_outputs;
    const SynBufferView* weights;
    size_t n_weights;
    SynSlice step;
    SynSlice workspace;
    const SynScalar* statics;
    size_t n_statics;
} SynOpArgs;

/* types.rs:294-306: the callee sets len and writes only when len <= cap */
typedef struct SynOutBuf {
    uint8_t* ptr;
    size_t cap;
    size_t len;
} SynOutBuf;

typedef struct SynRegistrarVtbl {
    uint32_t struct_size;
    SynStatus (*reg)(void* slf, SynHostRegion region, uint32_t flags, SynRegistration* out);
    SynStatus (*unreg)(void* slf, const SynRegistration* reg);
    SynStatus (*close)(void* slf);
    void* slf;
} SynRegistrarVtbl;

/* types.rs:336-536, in this order */
typedef struct SynProviderVtbl {
    uint32_t struct_size;
    const char* id;
    uint32_t backend;
    uint32_t domain;
    SynStatus (*build)(void* slf, SynOutBuf* out);
    SynStatus (*enumerate)(void* slf, SynOutBuf* out);
    SynStatus (*open)(void* slf, const SynDeviceId* dev, const SynOpenOptions* opts, uint64_t* ctx);
    SynStatus (*close_ctx)(void* slf, uint64_t ctx);
    SynStatus (*memory_info)(void* slf, uint64_t ctx, SynMemoryInfo* out);
    SynStatus (*ops)(void* slf, SynOutBuf* out);
    SynStatus (*query)(void* slf, uint64_t ctx, const uint8_t* op, size_t op_len,
                       const uint8_t* shape, size_t shape_len, SynOutBuf* out);
    SynStatus (*alloc)(void* slf, uint64_t ctx, const SynAllocRequest* req, SynBuffer* out);
    SynStatus (*free)(void* slf, uint64_t ctx, const SynBuffer* buf);
    SynStatus (*map_segment)(void* slf, uint64_t ctx, const SynBuffer* reservation,
                             uint64_t offset, uint64_t bytes, SynSegment* out);
    SynStatus (*unmap_segment)(void* slf, uint64_t ctx, const SynSegment* seg);
    SynStatus (*register_host)(void* slf, uint64_t ctx, SynHostRegion region,
                               SynRegistration* out);
    SynStatus (*host_registrar)(void* slf, uint64_t ctx, SynRegistrarVtbl* out);
    SynStatus (*import)(void* slf, uint64_t ctx, SynHostRegion region, SynBuffer* out);
    SynStatus (*set_resident)(void* slf, uint64_t ctx, const SynBuffer* bufs, size_t n,
                              uint32_t resident);
    SynStatus (*repack)(void* slf, const uint8_t* op, size_t op_len, const uint8_t* src,
                        size_t src_len, uint8_t* dst, size_t dst_len, uint32_t* present,
                        uint32_t* layout);
    SynStatus (*repacked_len)(void* slf, const uint8_t* op, size_t op_len, uint64_t src,
                              uint32_t* present, uint64_t* out);
    SynStatus (*stream)(void* slf, uint64_t ctx, uint32_t prio, uint64_t* out);
    SynStatus (*event)(void* slf, uint64_t ctx, uint64_t* out);
    SynStatus (*record)(void* slf, uint64_t ctx, uint64_t s, uint64_t e);
    SynStatus (*wait)(void* slf, uint64_t ctx, uint64_t s, uint64_t e);
    SynStatus (*signal_host)(void* slf, uint64_t ctx, uint64_t s, uint32_t flag, uint32_t value);
    SynStatus (*wait_host)(void* slf, uint64_t ctx, uint64_t s, uint32_t flag, uint32_t value,
                           uint32_t cmp, uint32_t has_reset, uint32_t reset);
    SynStatus (*arm_wake)(void* slf, uint64_t ctx, uint64_t s, uint32_t kind, uint64_t handle);
    SynStatus (*poll)(void* slf, uint64_t ctx, uint64_t e, uint32_t* done);
    SynStatus (*elapsed)(void* slf, uint64_t ctx, uint64_t start, uint64_t end, uint32_t* present,
                         uint64_t* nanos);
    SynStatus (*synchronize)(void* slf, uint64_t ctx, uint64_t s);
    SynStatus (*copy)(void* slf, uint64_t ctx, uint64_t s, const SynSlice* src, const SynSlice* dst);
    SynStatus (*copy_batch)(void* slf, uint64_t ctx, uint64_t s, const SynSlicePair* pairs, size_t n);
    SynStatus (*prepare)(void* slf, uint64_t ctx, const uint8_t* op, size_t op_len,
                         const uint8_t* shape, size_t shape_len, SynPreparedOp* out);
    SynStatus (*launch)(void* slf, uint64_t ctx, uint64_t s, const SynPreparedOp* op,
                        const SynOpArgs* args);
    SynStatus (*begin_capture)(void* slf, uint64_t ctx, uint64_t s);
    SynStatus (*end_capture)(void* slf, uint64_t ctx, uint64_t s, uint64_t* out);
    SynStatus (*replay)(void* slf, uint64_t ctx, uint64_t s, uint64_t g);
    SynStatus (*health)(void* slf, uint64_t ctx, SynHealth* out);
    SynStatus (*last_error)(void* slf, uint64_t ctx, uint8_t* buf, size_t cap, size_t* len);
    void* slf;
    uint32_t health_size;
} SynProviderVtbl;

/* types.rs:540-549 */
typedef struct SynModule {
    SynHeader h;
    uint32_t n_providers;
    const SynProviderVtbl* providers;
    SynStatus (*shutdown)(void);
} SynModule;

/* The entry point (crates/kernels/src/abi/mod.rs:64: ENTRY_SYMBOL; EntryFn).  Returns null when
 * the host's header is not "SYNPROV1", major 1, or shorter than this header's SynHostApi.  The
 * module has one provider: id "hip", backend Hip, domain Hip, serving Gemv, Gemm, Logits and
 * GateUpAct{Silu} (Q4_0, Q8_0, Q4_K, F16, BF16), MoeGrouped (Q4_K, Q8_0), MoeRoute{Softmax} and
 * MoeCombine on AMD gfx950 devices. */
const SynModule* syntropy_provider_entry_v1(const SynHostApi* host);

#ifdef __cplusplus
}
#endif

#endif /* SYNTROPY_PROVIDER_H */
