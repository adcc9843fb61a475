"""Host side of the provider-library boundary (include/syntropy_provider.h), in ctypes.

`load(path)` does what the reference core's loader does with a kernel module
(crates/kernels-loader/src/module.rs:94: dlopen, dlsym "syntropy_provider_entry_v1", call it with
the host's services, check the returned header), and `Provider` wraps one SynProviderVtbl the way
kernels_loader::ModuleProvider does (crates/kernels-loader/src/provider.rs): every entry returns a
SynStatus; a failure raises ProviderError with the entry's per-thread message; variable-size
results are fetched through a caller buffer and retried at the reported length; JSON records
(OpKey, ShapeSig, CapsWire) are serde's forms.
"""
from __future__ import annotations

import ctypes as C
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PROVIDER_LIB = os.path.join(HERE, "libsyntropy_provider.so")

MAGIC = b"SYNPROV1"
ABI_MAJOR, ABI_MINOR = 1, 0
HEALTH_SIZE = 12
BACKEND_HIP = MEMDOMAIN_HIP = 2
# DType::ALL indices (crates/core/src/dtype.rs:55-71)
DT_F32, DT_I32 = 0, 7
# MemKind (crates/kernels/src/memory.rs:33-40); doorbell pages are 4 KiB of HostMapped buffers
KIND_DEVICE, KIND_HOST_MAPPED = 0, 1
DOORBELL_PAGE = 4096
MAX_DOORBELL_PAGES = 1 << 16  # page numbers are 16 bits (HostFlag = page << 16 | slot)
# status classes and Kernels-domain codes (RFC-0040 13)
CLASS_DEVICE, CLASS_TIMEOUT, CLASS_INTERNAL = 6, 10, 13
CODE_DEVICE_STICKY, CODE_DOORBELL_TIMEOUT, CODE_PROVIDER_PANICKED = 8, 11, 16

u8, u16, u32, u64, sz, vp = C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64, C.c_size_t, C.c_void_p


class Header(C.Structure):
    _fields_ = [("magic", u8 * 8), ("abi_major", u32), ("abi_minor", u32), ("build_id", u8 * 32),
                ("struct_size", u32)]


class Status(C.Structure):
    _fields_ = [("cls", u32), ("domain", u32), ("code", u16), ("retry", u8)]


LOGFN = C.CFUNCTYPE(None, u8, C.c_char_p, C.c_void_p, sz)
METRICFN = C.CFUNCTYPE(None, u32, u64)
# returns a NUL-terminated string the host keeps alive, or null (a c_void_p: ctypes would free a
# returned bytes object)
CONFIGFN = C.CFUNCTYPE(C.c_void_p, C.c_char_p)


class HostApi(C.Structure):
    _fields_ = [("h", Header), ("log", LOGFN), ("metric", METRICFN), ("config", CONFIGFN)]


class DeviceId(C.Structure):
    _fields_ = [("node", u8 * 32), ("ordinal", u32)]


class OpenOptions(C.Structure):
    _fields_ = [("streams", u8 * 4), ("doorbell_slots", u32), ("capture", u8), ("deterministic", u8),
                ("power", u8), ("reserved", u8)]


class MemoryInfo(C.Structure):
    _fields_ = [("total", u64), ("free", u64), ("budget", u64), ("host_visible", u64),
                ("max_alloc", u64), ("flags", u32), ("reserved", u32)]


class AllocRequest(C.Structure):
    _fields_ = [("bytes", u64), ("align", u64), ("kind", u32), ("reserve_only", u32)]


class Buffer(C.Structure):
    _fields_ = [("addr", u64), ("bytes", u64), ("handle", u64), ("kind", u32), ("reserved", u32)]


class Slice(C.Structure):
    _fields_ = [("buffer", u64), ("offset", u64), ("bytes", u64)]


class SlicePair(C.Structure):
    _fields_ = [("src", Slice), ("dst", Slice)]


class HostRegion(C.Structure):
    _fields_ = [("addr", u64), ("len", u64)]


class Health(C.Structure):
    _fields_ = [("kind", u32), ("domain", u32), ("detail", u32)]


class PreparedOp(C.Structure):
    _fields_ = [("workspace", u64), ("handle", u64)]


class TensorArg(C.Structure):
    _fields_ = [("buf", Slice), ("dtype", u32), ("reserved", u32), ("dims", u32 * 4),
                ("strides", u32 * 4)]


class BufferView(C.Structure):
    _fields_ = [("kind", u32), ("ordinal", u32), ("node", u8 * 32), ("addr", u64), ("len", u64)]


class Scalar(C.Structure):
    _fields_ = [("tag", u32), ("bits", u32)]


class OpArgs(C.Structure):
    _fields_ = [("struct_size", u32), ("has_workspace", u32), ("inputs", C.POINTER(TensorArg)),
                ("n_inputs", sz), ("outputs", C.POINTER(TensorArg)), ("n_outputs", sz),
                ("weights", C.POINTER(BufferView)), ("n_weights", sz), ("step", Slice),
                ("workspace", Slice), ("statics", C.POINTER(Scalar)), ("n_statics", sz)]


class OutBuf(C.Structure):
    _fields_ = [("ptr", C.POINTER(u8)), ("cap", sz), ("len", sz)]


S = Status
_P = C.POINTER
VTBL_FUNCS = [
    ("build", [vp, _P(OutBuf)]),
    ("enumerate", [vp, _P(OutBuf)]),
    ("open", [vp, _P(DeviceId), _P(OpenOptions), _P(u64)]),
    ("close_ctx", [vp, u64]),
    ("memory_info", [vp, u64, _P(MemoryInfo)]),
    ("ops", [vp, _P(OutBuf)]),
    ("query", [vp, u64, _P(u8), sz, _P(u8), sz, _P(OutBuf)]),
    ("alloc", [vp, u64, _P(AllocRequest), _P(Buffer)]),
    ("free", [vp, u64, _P(Buffer)]),
    ("map_segment", [vp, u64, _P(Buffer), u64, u64, vp]),
    ("unmap_segment", [vp, u64, vp]),
    ("register_host", [vp, u64, HostRegion, vp]),
    ("host_registrar", [vp, u64, vp]),
    ("import", [vp, u64, HostRegion, _P(Buffer)]),
    ("set_resident", [vp, u64, _P(Buffer), sz, u32]),
    ("repack", [vp, _P(u8), sz, _P(u8), sz, _P(u8), sz, _P(u32), _P(u32)]),
    ("repacked_len", [vp, _P(u8), sz, u64, _P(u32), _P(u64)]),
    ("stream", [vp, u64, u32, _P(u64)]),
    ("event", [vp, u64, _P(u64)]),
    ("record", [vp, u64, u64, u64]),
    ("wait", [vp, u64, u64, u64]),
    ("signal_host", [vp, u64, u64, u32, u32]),
    ("wait_host", [vp, u64, u64, u32, u32, u32, u32, u32]),
    ("arm_wake", [vp, u64, u64, u32, u64]),
    ("poll", [vp, u64, u64, _P(u32)]),
    ("elapsed", [vp, u64, u64, u64, _P(u32), _P(u64)]),
    ("synchronize", [vp, u64, u64]),
    ("copy", [vp, u64, u64, _P(Slice), _P(Slice)]),
    ("copy_batch", [vp, u64, u64, _P(SlicePair), sz]),
    ("prepare", [vp, u64, _P(u8), sz, _P(u8), sz, _P(PreparedOp)]),
    ("launch", [vp, u64, u64, _P(PreparedOp), _P(OpArgs)]),
    ("begin_capture", [vp, u64, u64]),
    ("end_capture", [vp, u64, u64, _P(u64)]),
    ("replay", [vp, u64, u64, u64]),
    ("health", [vp, u64, _P(Health)]),
    ("last_error", [vp, u64, _P(u8), sz, _P(sz)]),
]


class Vtbl(C.Structure):
    _fields_ = ([("struct_size", u32), ("id", C.c_char_p), ("backend", u32), ("domain", u32)] +
                [(n, C.CFUNCTYPE(Status, *a)) for n, a in VTBL_FUNCS] +
                [("slf", vp), ("health_size", u32)])


class Module(C.Structure):
    _fields_ = [("h", Header), ("n_providers", u32), ("providers", C.POINTER(Vtbl)),
                ("shutdown", C.CFUNCTYPE(Status))]


class ProviderError(RuntimeError):
    """A failed entry: the SynStatus fields and the provider's message."""

    def __init__(self, entry: str, st: Status, message: str):
        super().__init__(f"{entry}: class {st.cls} code {st.code}: {message}")
        self.entry, self.cls, self.code, self.domain = entry, st.cls, st.code, st.domain
        self.message = message


# The host's services, as the core's loader provides them (crates/kernels-loader/src/host.rs):
# process-wide and alive for the module's life.  CONFIG holds the config keys the module reads
# (kernels.spin_kernel_max_us, and the fault-injection keys fixture.panic_in and
# fixture.device_fault_in, which the module reads once, at its entry); LOG collects
# (level, target, message) of every log call.
CONFIG: dict = {}
LOG: list = []
_config_strings: dict = {}


def _log(level, target, msg, n):
    LOG.append((int(level), target.decode(errors="replace"), C.string_at(msg, n).decode(errors="replace")))


def _metric(i, v):
    return None


def _config(key):
    v = CONFIG.get(key.decode())
    if v is None:
        return None
    buf = _config_strings.setdefault(v, C.create_string_buffer(str(v).encode()))
    return C.addressof(buf)


_CALLBACKS = (LOGFN(_log), METRICFN(_metric), CONFIGFN(_config))


def host_api(magic: bytes = MAGIC, major: int = ABI_MAJOR, size: int | None = None) -> HostApi:
    """The host's services with a header of this library's identity (zero build id)."""
    h = Header()
    C.memmove(h.magic, magic, 8)
    h.abi_major, h.abi_minor = major, ABI_MINOR
    h.struct_size = C.sizeof(HostApi) if size is None else size
    return HostApi(h, *_CALLBACKS)


_HOST = host_api()


def load(path: str = PROVIDER_LIB, host: HostApi | None = None):
    """(Module pointer or None, the loaded library, the host api kept alive)."""
    lib = C.CDLL(path)
    entry = lib.syntropy_provider_entry_v1
    entry.argtypes = [C.POINTER(HostApi)]
    entry.restype = C.POINTER(Module)
    host = host if host is not None else _HOST
    m = entry(C.byref(host))
    return (m.contents if m else None), lib, host


def _bytes(s: str):
    b = s.encode()
    return (u8 * max(1, len(b))).from_buffer_copy(b or b"\0"), len(b)


class Provider:
    """One SynProviderVtbl, wrapped as the core's ModuleProvider wraps it."""

    def __init__(self, path: str = PROVIDER_LIB):
        m, self.lib, self.host = load(path)
        if m is None:
            raise RuntimeError("the module refused the host's header")
        if bytes(m.h.magic) != MAGIC or m.h.abi_major != ABI_MAJOR or m.h.struct_size < C.sizeof(Module):
            raise RuntimeError("the module's header is not this ABI's")
        if m.n_providers != 1:
            raise RuntimeError(f"{m.n_providers} providers in the module")
        self.module = m
        self.vt = m.providers[0]
        self._pages = {}  # per context: the next doorbell page number
        if self.vt.health_size != HEALTH_SIZE:
            raise RuntimeError("health_size is not 12")

    # -- plumbing --
    def message(self, ctx: int = 0) -> str:
        n = sz(0)
        self.vt.last_error(self.vt.slf, ctx, None, 0, C.byref(n))
        buf = (u8 * max(1, n.value))()
        self.vt.last_error(self.vt.slf, ctx, buf, n.value, C.byref(n))
        return bytes(buf[: n.value]).decode(errors="replace")

    def _ok(self, name: str, st: Status, ctx: int = 0):
        if st.cls != 0:
            raise ProviderError(name, st, self.message(ctx))

    def _fetch(self, name: str, fn, *args, ctx: int = 0) -> bytes:
        cap = 256
        while True:
            buf = (u8 * cap)()
            out = OutBuf(C.cast(buf, C.POINTER(u8)), cap, 0)
            self._ok(name, fn(self.vt.slf, *args, C.byref(out)), ctx)
            if out.len <= cap:
                return bytes(buf[: out.len])
            cap = out.len

    # -- entries --
    def id(self) -> str:
        return self.vt.id.decode()

    def build(self) -> dict:
        return json.loads(self._fetch("build", self.vt.build))

    def enumerate(self) -> list:
        return json.loads(self._fetch("enumerate", self.vt.enumerate))

    def ops(self) -> list:
        return json.loads(self._fetch("ops", self.vt.ops))

    def open(self, ordinal: int = 0, doorbell_slots: int = 0) -> int:
        dev, opts, ctx = DeviceId(), OpenOptions(), u64(0)
        dev.ordinal = ordinal
        opts.doorbell_slots = doorbell_slots
        self._ok("open", self.vt.open(self.vt.slf, C.byref(dev), C.byref(opts), C.byref(ctx)))
        return ctx.value

    def close(self, ctx: int):
        self._ok("close_ctx", self.vt.close_ctx(self.vt.slf, ctx), ctx)

    def memory_info(self, ctx: int) -> MemoryInfo:
        m = MemoryInfo()
        self._ok("memory_info", self.vt.memory_info(self.vt.slf, ctx, C.byref(m)), ctx)
        return m

    def query(self, ctx: int, op: dict, shape: dict) -> dict | None:
        (ob, on), (sb, sn) = _bytes(json.dumps(op)), _bytes(json.dumps(shape))
        raw = self._fetch("query", self.vt.query, ctx, ob, on, sb, sn, ctx=ctx)
        return json.loads(raw) if raw else None

    def prepare(self, ctx: int, op: dict, shape: dict) -> PreparedOp:
        (ob, on), (sb, sn) = _bytes(json.dumps(op)), _bytes(json.dumps(shape))
        p = PreparedOp()
        self._ok("prepare", self.vt.prepare(self.vt.slf, ctx, ob, on, sb, sn, C.byref(p)), ctx)
        return p

    def alloc(self, ctx: int, nbytes: int, align: int = 256, kind: int = KIND_DEVICE) -> Buffer:
        b = Buffer()
        self._ok("alloc", self.vt.alloc(self.vt.slf, ctx, C.byref(AllocRequest(nbytes, align, kind, 0)),
                                        C.byref(b)), ctx)
        if kind == KIND_HOST_MAPPED:  # the core numbers the doorbell pages in allocation order
            n, pages = self._pages.get(ctx, 0), -(-nbytes // DOORBELL_PAGE)
            if n + pages <= MAX_DOORBELL_PAGES:
                b.first_page = n
                self._pages[ctx] = n + pages
            else:  # allocated with no page numbers: its words hold no flags
                b.first_page = None
        return b

    def free(self, ctx: int, b: Buffer):
        self._ok("free", self.vt.free(self.vt.slf, ctx, C.byref(b)), ctx)

    def stream(self, ctx: int, prio: int = 0) -> int:
        s = u64(0)
        self._ok("stream", self.vt.stream(self.vt.slf, ctx, prio, C.byref(s)), ctx)
        return s.value

    def event(self, ctx: int) -> int:
        e = u64(0)
        self._ok("event", self.vt.event(self.vt.slf, ctx, C.byref(e)), ctx)
        return e.value

    def record(self, ctx: int, s: int, e: int):
        self._ok("record", self.vt.record(self.vt.slf, ctx, s, e), ctx)

    def elapsed(self, ctx: int, start: int, end: int):
        """Nanoseconds between two recorded events, or None when they hold no timing."""
        present, ns = u32(0), u64(0)
        self._ok("elapsed", self.vt.elapsed(self.vt.slf, ctx, start, end, C.byref(present), C.byref(ns)), ctx)
        return ns.value if present.value else None

    def poll(self, ctx: int, e: int) -> bool:
        d = u32(0)
        self._ok("poll", self.vt.poll(self.vt.slf, ctx, e, C.byref(d)), ctx)
        return bool(d.value)

    def synchronize(self, ctx: int, s: int):
        self._ok("synchronize", self.vt.synchronize(self.vt.slf, ctx, s), ctx)

    def copy(self, ctx: int, s: int, src: Slice, dst: Slice):
        self._ok("copy", self.vt.copy(self.vt.slf, ctx, s, C.byref(src), C.byref(dst)), ctx)

    def launch(self, ctx: int, s: int, op: PreparedOp, args: OpArgs):
        self._ok("launch", self.vt.launch(self.vt.slf, ctx, s, C.byref(op), C.byref(args)), ctx)

    def begin_capture(self, ctx: int, s: int):
        self._ok("begin_capture", self.vt.begin_capture(self.vt.slf, ctx, s), ctx)

    def end_capture(self, ctx: int, s: int) -> int:
        g = u64(0)
        self._ok("end_capture", self.vt.end_capture(self.vt.slf, ctx, s, C.byref(g)), ctx)
        return g.value

    def replay(self, ctx: int, s: int, g: int):
        self._ok("replay", self.vt.replay(self.vt.slf, ctx, s, g), ctx)

    # -- doorbells (provider.rs:346-377; RFC-0040 4.2) --
    def signal_host(self, ctx: int, s: int, page: int, slot: int, value: int = 1):
        self._ok("signal_host", self.vt.signal_host(self.vt.slf, ctx, s, page << 16 | slot, value), ctx)

    def wait_host(self, ctx: int, s: int, page: int, slot: int, value: int = 1, geq: bool = False,
                  reset: int | None = 0):
        self._ok("wait_host", self.vt.wait_host(self.vt.slf, ctx, s, page << 16 | slot, value, int(geq),
                                                int(reset is not None), reset or 0), ctx)

    def arm_wake(self, ctx: int, s: int, kind: int, handle: int):
        """After the work enqueued so far on `s`, wake a host thread without `s` waiting:
        kind 0 a futex word's address (cleared from 1 and woken), kind 1 an eventfd (+1)."""
        self._ok("arm_wake", self.vt.arm_wake(self.vt.slf, ctx, s, kind, handle), ctx)

    def health(self, ctx: int = 0) -> Health:
        h = Health()
        self._ok("health", self.vt.health(self.vt.slf, ctx, C.byref(h)), ctx)
        return h


def host_flag(buf: Buffer, offset: int):
    """(page, slot) of the doorbell flag at byte `offset` of a HostMapped buffer, and the host's
    c_uint32 over it (the buffer's addr is also its host address)."""
    assert offset % 4 == 0 and 0 <= offset < buf.bytes
    if buf.first_page is None:
        raise ValueError("the buffer's pages carry no doorbell numbers")
    page = buf.first_page + offset // DOORBELL_PAGE
    slot = offset % DOORBELL_PAGE // 4
    return page, slot, u32.from_address(buf.addr + offset)


def packed(buf: Buffer, dtype: int, dims, offset: int = 0, elem: int = 4) -> TensorArg:
    """A packed tensor argument over `buf` (crates/kernels/src/op/args.rs:85-96)."""
    d = list(dims) + [1] * (4 - len(dims))
    st = [1, 1, 1, 1]
    for i in (2, 1, 0):
        st[i] = st[i + 1] * d[i + 1]
    n = d[0] * d[1] * d[2] * d[3] * elem
    return TensorArg(Slice(buf.handle, offset, n), dtype, 0, (u32 * 4)(*d), (u32 * 4)(*st))


def op_args(inputs, outputs, weights, workspace: Slice | None = None, statics=(),
            step: Slice | None = None) -> OpArgs:
    """SynOpArgs (types.rs:267-292).  `step` is the step descriptor's slice (its rows_active
    bounds the rows computed); none computes the whole bucket."""
    ins = (TensorArg * max(1, len(inputs)))(*inputs)
    outs = (TensorArg * max(1, len(outputs)))(*outputs)
    ws = (BufferView * max(1, len(weights)))(*weights)
    st = (Scalar * max(1, len(statics)))(*statics)
    a = OpArgs(C.sizeof(OpArgs), 1 if workspace is not None else 0, ins, len(inputs), outs, len(outputs),
               ws, len(weights), step or Slice(), workspace or Slice(), st, len(statics))
    a._keep = (ins, outs, ws, st)
    return a


def view(addr: int, nbytes: int) -> BufferView:
    v = BufferView()
    v.addr, v.len = addr, nbytes
    return v


__all__ = ["Provider", "ProviderError", "load", "host_api", "host_flag", "packed", "op_args", "view",
           "Slice", "Buffer", "PreparedOp", "Scalar", "DT_F32", "DT_I32", "PROVIDER_LIB", "MAGIC", "CONFIG",
           "LOG", "KIND_DEVICE", "KIND_HOST_MAPPED"]
