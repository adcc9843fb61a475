"""Doorbells through the provider boundary (crates/kernels/src/provider.rs:346-377; RFC-0040 4.2
and its 2026-11-07 revision): flags are 4-byte words of the 4 KiB pages of HostMapped buffers
the host allocated through `alloc`, numbered in allocation order.  signal_host raises a flag
after the work before it, wait_host holds the stream until the host replies and then writes the
consumer reset, a captured step runs the constant-valued handshake on every replay, and a wait
that passes its spin limit ends on its own and is reported as a DoorbellTimeout.  Every wait here
is answered by the host except the one that tests the limit, which runs on a context opened with
kernels.spin_kernel_max_us = 2000.  Each flag sits on a 64-byte line of its own, as the host's
rule asks (RFC-0040 4.2)."""
import os
import time

import numpy as np
import pytest

from gpu_util import announce
from oracle import oracle as o
from refgen import GemvRng, gemv_activations, gemv_weights
from test_gpu_provider import Ctx, gemv_key, shape

pytestmark = pytest.mark.gpu

N_OUT, K, ROWS = 512, 1024, 2


@pytest.fixture(scope="module")
def cx():
    c = Ctx()
    c.bells = c.pr.alloc(c.ctx, 4096, kind=c.P.KIND_HOST_MAPPED)
    yield c
    c.close()


def bell(cx, i):
    """Flag i of the context's doorbell buffer: (page, slot, host word), on line i."""
    return cx.P.host_flag(cx.bells, 64 * i)


def gemv_step(cx, seed):
    """A prepared Q4_K Gemv with its buffers: (launch args, x buffer, y buffer, weights)."""
    P, pr = cx.P, cx.pr
    rng = GemvRng(seed)
    w = gemv_weights(rng, o.Q4_K, N_OUT, K, o.f16_bits, o.round_bf16)
    op = pr.prepare(cx.ctx, gemv_key(o.Q4_K), shape(ROWS, N_OUT, K))
    wb = cx.put(w)
    xb, yb = cx.empty(4 * ROWS * K, 0), cx.empty(4 * ROWS * N_OUT)
    args = P.op_args([P.packed(xb, P.DT_F32, [ROWS, K])], [P.packed(yb, P.DT_F32, [ROWS, N_OUT])],
                     [P.view(wb.addr, w.nbytes)], cx.workspace(op))
    return op, args, xb, yb, w, rng


def wait_for(flag, value, seconds=5.0):
    end = time.monotonic() + seconds
    while flag.value != value:
        if time.monotonic() > end:
            return False
        time.sleep(0.0005)
    return True


def test_signal_host_follows_the_work_before_it(cx):
    pr = cx.pr
    op, args, xb, yb, w, rng = gemv_step(cx, 1)
    x = gemv_activations(rng, ROWS, K).reshape(ROWS, K).astype(np.float32)
    cx.upload(xb.addr, x)
    page, slot, flag = bell(cx, 1)
    flag.value = 0
    announce("signal_host")
    pr.launch(cx.ctx, cx.s, op, args)
    pr.signal_host(cx.ctx, cx.s, page, slot, 1)
    assert wait_for(flag, 1)
    pr.synchronize(cx.ctx, cx.s)
    got = cx.get(yb, np.float32, (ROWS, N_OUT))
    assert (got.view(np.uint32) == o.gemv(o.Q4_K, w, N_OUT, K, x, ROWS).view(np.uint32)).all()
    flag.value = 0


def test_wait_host_holds_the_stream_until_the_host_replies(cx):
    """wait_host(Eq 1, reset 0) -> Gemv -> signal_host: the done flag stays down while the host
    has not replied, then rises; the reply flag is back at 0 and the output is the oracle's."""
    pr = cx.pr
    op, args, xb, yb, w, rng = gemv_step(cx, 2)
    x = gemv_activations(rng, ROWS, K).reshape(ROWS, K).astype(np.float32)
    cx.upload(xb.addr, x)
    (rp, rs, reply), (dp, ds, done) = bell(cx, 2), bell(cx, 3)
    reply.value, done.value = 0, 0
    announce("wait_host handshake")
    pr.wait_host(cx.ctx, cx.s, rp, rs, 1, reset=0)
    pr.launch(cx.ctx, cx.s, op, args)
    pr.signal_host(cx.ctx, cx.s, dp, ds, 1)
    time.sleep(0.1)
    held = done.value
    reply.value = 1
    assert wait_for(done, 1)
    pr.synchronize(cx.ctx, cx.s)
    assert held == 0, "the stream ran past wait_host before the host replied"
    assert reply.value == 0, "the consumer reset was not written"
    got = cx.get(yb, np.float32, (ROWS, N_OUT))
    assert (got.view(np.uint32) == o.gemv(o.Q4_K, w, N_OUT, K, x, ROWS).view(np.uint32)).all()
    done.value = 0


def test_wait_host_geq_and_no_reset(cx):
    pr = cx.pr
    (rp, rs, reply), (dp, ds, done) = bell(cx, 4), bell(cx, 5)
    reply.value, done.value = 3, 0
    announce("wait_host geq")
    pr.wait_host(cx.ctx, cx.s, rp, rs, 5, geq=True, reset=None)
    pr.signal_host(cx.ctx, cx.s, dp, ds, 1)
    time.sleep(0.05)
    held = done.value
    reply.value = 9
    assert wait_for(done, 1)
    pr.synchronize(cx.ctx, cx.s)
    assert held == 0 and reply.value == 9
    done.value = 0


def test_captured_step_runs_the_handshake_on_every_replay(cx):
    """One capture of wait_host(F = 1, reset 0) -> Gemv -> signal_host(D, 1), replayed three
    times: per step the host writes x, raises F, waits for D, resets D (RFC-0040 4.2 rules 2-3)."""
    pr = cx.pr
    op, args, xb, yb, w, rng = gemv_step(cx, 3)
    (fp, fs, f), (dp, ds, d) = bell(cx, 6), bell(cx, 7)
    f.value, d.value = 0, 0
    announce("doorbell capture/replay")
    pr.begin_capture(cx.ctx, cx.s)
    pr.wait_host(cx.ctx, cx.s, fp, fs, 1, reset=0)
    pr.launch(cx.ctx, cx.s, op, args)
    pr.signal_host(cx.ctx, cx.s, dp, ds, 1)
    g = pr.end_capture(cx.ctx, cx.s)
    for step in range(3):
        x = gemv_activations(rng, ROWS, K).reshape(ROWS, K).astype(np.float32)
        cx.upload(xb.addr, x)
        pr.replay(cx.ctx, cx.s, g)
        time.sleep(0.02)
        assert d.value == 0, f"step {step}: done before the reply"
        f.value = 1
        assert wait_for(d, 1), f"step {step}: no done flag"
        d.value = 0
        pr.synchronize(cx.ctx, cx.s)
        assert f.value == 0
        got = cx.get(yb, np.float32, (ROWS, N_OUT))
        assert (got.view(np.uint32) == o.gemv(o.Q4_K, w, N_OUT, K, x, ROWS).view(np.uint32)).all(), step


def wait_readable(fd, seconds=5.0):
    import select
    r, _, _ = select.select([fd], [], [], seconds)
    return bool(r)


def test_arm_wake_eventfd_after_the_doorbell(cx):
    """arm_wake after signal_host: the eventfd fires once the doorbell is up (the wake follows
    the work before it) and the stream did not wait for it."""
    pr = cx.pr
    op, args, xb, yb, w, rng = gemv_step(cx, 4)
    cx.upload(xb.addr, gemv_activations(rng, ROWS, K).reshape(ROWS, K).astype(np.float32))
    dp, ds, d = bell(cx, 11)
    d.value = 0
    fd = os.eventfd(0, os.EFD_NONBLOCK)
    try:
        announce("arm_wake eventfd")
        pr.launch(cx.ctx, cx.s, op, args)
        pr.signal_host(cx.ctx, cx.s, dp, ds, 1)
        pr.arm_wake(cx.ctx, cx.s, 1, fd)
        assert wait_readable(fd), "no wake within 5 s"
        assert d.value == 1, "the wake came before the doorbell"
        assert os.eventfd_read(fd) == 1
        pr.synchronize(cx.ctx, cx.s)
        # many wakes of one target reuse the context's fork event and target record
        for _ in range(100):
            pr.arm_wake(cx.ctx, cx.s, 1, fd)
        pr.synchronize(cx.ctx, cx.s)
        end = time.monotonic() + 5
        n = 0
        while n < 100 and time.monotonic() < end:
            if wait_readable(fd, 0.5):
                n += os.eventfd_read(fd)
        assert n == 100
    finally:
        os.close(fd)
        d.value = 0


def test_arm_wake_futex_word_is_cleared_and_woken(cx):
    """A futex word the waiter armed (1) is cleared by the wake, and a thread waiting on it in
    FUTEX_WAIT returns before its timeout."""
    import ctypes as C
    import threading
    pr = cx.pr
    word = C.c_uint32(1)
    libc = C.CDLL(None, use_errno=True)

    class Timespec(C.Structure):
        _fields_ = [("tv_sec", C.c_long), ("tv_nsec", C.c_long)]

    out = {}

    def waiter():
        t0 = time.monotonic()
        rc = libc.syscall(202, C.byref(word), 0, 1, C.byref(Timespec(5, 0)), None, 0)  # FUTEX_WAIT on 1
        out["rc"], out["errno"], out["dt"] = rc, C.get_errno(), time.monotonic() - t0

    th = threading.Thread(target=waiter)
    th.start()
    time.sleep(0.05)  # the waiter is in FUTEX_WAIT (or returns EAGAIN if the wake came first)
    announce("arm_wake futex")
    pr.arm_wake(cx.ctx, cx.s, 0, C.addressof(word))
    th.join(10)
    pr.synchronize(cx.ctx, cx.s)
    assert word.value == 0
    assert out["dt"] < 4.5, "the waiter slept until its timeout"
    assert out["rc"] == 0 or out["errno"] == 11  # woken, or the word was already cleared


def test_captured_arm_wake_fires_on_every_replay(cx):
    pr = cx.pr
    op, args, xb, yb, w, rng = gemv_step(cx, 5)
    dp, ds, d = bell(cx, 12)
    d.value = 0
    fd = os.eventfd(0, os.EFD_NONBLOCK)
    try:
        announce("arm_wake capture/replay")
        pr.begin_capture(cx.ctx, cx.s)
        pr.launch(cx.ctx, cx.s, op, args)
        pr.signal_host(cx.ctx, cx.s, dp, ds, 1)
        pr.arm_wake(cx.ctx, cx.s, 1, fd)
        g = pr.end_capture(cx.ctx, cx.s)
        for step in range(3):
            x = gemv_activations(rng, ROWS, K).reshape(ROWS, K).astype(np.float32)
            cx.upload(xb.addr, x)
            pr.replay(cx.ctx, cx.s, g)
            assert wait_readable(fd), f"replay {step}: no wake"
            assert d.value == 1 and os.eventfd_read(fd) == 1, step
            d.value = 0
            pr.synchronize(cx.ctx, cx.s)
            got = cx.get(yb, np.float32, (ROWS, N_OUT))
            assert (got.view(np.uint32) == o.gemv(o.Q4_K, w, N_OUT, K, x, ROWS).view(np.uint32)).all(), step
    finally:
        os.close(fd)


def test_pages_are_numbered_in_allocation_order(cx):
    """Pages count across the context's HostMapped buffers in allocation order and are never
    renumbered; a flag outside a live page, past a page or past its buffer's end is refused
    before anything is enqueued; device memory holds no flags
    (crates/kernels-cuda/src/capture/tests.rs:416-456)."""
    P, pr = cx.P, cx.pr
    big = pr.alloc(cx.ctx, 3 * 4096, kind=P.KIND_HOST_MAPPED)
    short = pr.alloc(cx.ctx, 100, kind=P.KIND_HOST_MAPPED)
    assert big.first_page == cx.bells.first_page + 1 and short.first_page == big.first_page + 3
    assert big.addr % 4096 == 0 and big.kind == P.KIND_HOST_MAPPED
    page, slot, w = P.host_flag(big, 2 * 4096 + 8)
    assert (page, slot) == (big.first_page + 2, 2)
    w.value = 0
    announce("doorbell page numbering")
    pr.signal_host(cx.ctx, cx.s, page, slot, 7)
    pr.synchronize(cx.ctx, cx.s)
    assert w.value == 7
    sp, ss, sw = P.host_flag(short, 96)  # the last whole word of the 100-byte buffer
    pr.signal_host(cx.ctx, cx.s, sp, ss, 3)
    pr.synchronize(cx.ctx, cx.s)
    assert sw.value == 3
    refused = [(short.first_page, 25),           # past the buffer's end
               (cx.bells.first_page, 1024),      # past the page
               (short.first_page + 1, 0),        # no such page yet
               (65535, 0)]
    pr.free(cx.ctx, big)
    refused += [(big.first_page, 0), (big.first_page + 2, 2)]  # freed pages
    for page, slot in refused:
        with pytest.raises(P.ProviderError) as e:
            pr.signal_host(cx.ctx, cx.s, page, slot, 1)
        assert e.value.cls == P.CLASS_INTERNAL and f"page {page} slot {slot}" in e.value.message
        with pytest.raises(P.ProviderError):
            pr.wait_host(cx.ctx, cx.s, page, slot, 1)
    nxt = pr.alloc(cx.ctx, 4096, kind=P.KIND_HOST_MAPPED)
    assert nxt.first_page == short.first_page + 1  # freed numbers are not reused
    pr.signal_host(cx.ctx, cx.s, short.first_page, 0, 1)  # the short buffer's flags still work
    pr.synchronize(cx.ctx, cx.s)
    pr.free(cx.ctx, short)
    pr.free(cx.ctx, nxt)


def test_page_numbers_run_out_without_failing_alloc():
    """A HostMapped buffer of n bytes takes ceil(n / 4096) page numbers, none for 0 bytes; one
    whose pages would pass number 65535 is still allocated, with no numbers, and leaves the count
    where it was (crates/kernels-cuda/src/memory.rs:546-559).  On a context of its own: it spends
    every number."""
    cx = Ctx()
    P, pr = cx.P, cx.pr
    empty = pr.alloc(cx.ctx, 0, kind=P.KIND_HOST_MAPPED)
    one = pr.alloc(cx.ctx, 4096, kind=P.KIND_HOST_MAPPED)
    assert one.first_page == empty.first_page  # the empty buffer took no number
    nxt = one.first_page + 1
    announce("doorbell page numbers past 65535")
    too_big = pr.alloc(cx.ctx, (65536 - nxt + 1) * 4096, kind=P.KIND_HOST_MAPPED)  # one page too many
    assert too_big.first_page is None and too_big.addr % 4096 == 0
    with pytest.raises(P.ProviderError):
        pr.signal_host(cx.ctx, cx.s, nxt, 0, 1)  # no page took that number
    pr.free(cx.ctx, too_big)
    fits = pr.alloc(cx.ctx, (65536 - nxt) * 4096, kind=P.KIND_HOST_MAPPED)  # exactly the rest
    assert fits.first_page == nxt
    page, slot, w = P.host_flag(fits, fits.bytes - 4)
    assert (page, slot) == (65535, 1023)
    w.value = 0
    pr.signal_host(cx.ctx, cx.s, page, slot, 5)
    pr.synchronize(cx.ctx, cx.s)
    assert w.value == 5
    after = pr.alloc(cx.ctx, 4096, kind=P.KIND_HOST_MAPPED)  # numbers spent: still allocated
    assert after.first_page is None and after.addr != 0
    for b in (empty, one, fits, after):
        pr.free(cx.ctx, b)
    cx.close()


def test_a_wait_past_its_spin_limit_ends_and_is_reported():
    """A context opened with kernels.spin_kernel_max_us = 2000: a wait the host never answers
    gives up on its own, writes no reset, lets the stream run on (the next flag rises), and
    synchronize reports one Timeout / DoorbellTimeout (11) naming the flag; the next synchronize
    is clean (RFC-0040 ...md:1342, 1361)."""
    from syntropy_amd import provider as P
    P.CONFIG["kernels.spin_kernel_max_us"] = "2000"
    try:
        c = Ctx()
    finally:
        del P.CONFIG["kernels.spin_kernel_max_us"]
    try:
        pr = c.pr
        b = pr.alloc(c.ctx, 4096, kind=P.KIND_HOST_MAPPED)
        (rp, rs, reply), (ap, as_, after) = P.host_flag(b, 9 * 64), P.host_flag(b, 10 * 64)
        reply.value, after.value = 0, 0
        announce("wait_host spin limit 2 ms")
        pr.wait_host(c.ctx, c.s, rp, rs, 1, reset=5)
        pr.signal_host(c.ctx, c.s, ap, as_, 1)
        with pytest.raises(P.ProviderError) as e:
            pr.synchronize(c.ctx, c.s)
        assert (e.value.cls, e.value.code) == (P.CLASS_TIMEOUT, P.CODE_DOORBELL_TIMEOUT)
        assert f"page {rp} slot {rs}" in str(e.value) and "spin limit of 2000" in str(e.value)
        assert reply.value == 0 and after.value == 1
        pr.synchronize(c.ctx, c.s)
    finally:
        c.close()
