"""The allocation-free design entry point through the C ABI.

hkbs_pmpnn_design_device_noalloc runs the kernels of hkbs_pmpnn_design_device
with its scratch in one static device array per GPU, so its outputs must be
bit-identical to that entry point's on the same inputs. Two calls in a row (the
second smaller, with per-sequence orders, chain labels and residue offsets)
check that what the first call leaves in the shared array does not leak into
the second; an oversized request is refused before any GPU work. A call leaves
the device's free memory unchanged, and the call captured on a caller's stream
into a HIP graph replays to the same bits, with other work between replays.
"""
import ctypes as C

import numpy as np
import pytest

from hikoboshi_amd import _lib, backbone, hip

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _dev(a):
    return None if a is None else hip.DeviceBuffer.from_array(a)


def _host(buf, shape, dtype):
    out = np.empty(shape, dtype)
    hip.check(hip.rt().hipMemcpy(out.ctypes.data_as(C.c_void_p), buf.ptr, C.c_size_t(out.nbytes), hip.D2H), "D2H")
    return out


def _design(ctx, entry, bb, B, orders, shared, seeds, T):
    """One call of `entry` (a C-ABI function name) on device buffers; returns host copies of the outputs."""
    lib = _lib.load()
    L = bb.L
    ins = [_dev(bb.coords), _dev(bb.atom_sources), _dev(bb.residue_indices), _dev(bb.chain_labels),
           _dev(orders), _dev(seeds)]
    outs = [hip.DeviceBuffer(B * L * 4), hip.DeviceBuffer(B * L * 21 * 4), hip.DeviceBuffer(B * 4)]
    for o in outs:  # stale values must not survive a call
        hip.check(hip.rt().hipMemset(o.ptr, 0xFF, C.c_size_t(o.nbytes)), "memset")
    c, s, r, ch, od, sd = ins
    _lib.check(getattr(lib, entry)(ctx._h, c.ptr, s.ptr, r.ptr if r else None, ch.ptr if ch else None, None, None,
                                   L, B, od.ptr, int(shared), sd.ptr, C.c_float(T), 0, outs[0].ptr, outs[1].ptr,
                                   outs[2].ptr, None))
    hip.device_synchronize()
    return (_host(outs[0], (B, L), np.int32), _host(outs[1], (B, L, 21), np.float32),
            _host(outs[2], (B,), np.float32))


def test_noalloc_design_matches_device_design(gpu_ctx):
    big = backbone.single_chain(300, 7)
    big_order = _lib.decode_order(big.atom_sources, 7)
    big_seeds = (7 + np.arange(16)).astype(np.uint64)
    small = backbone.tetrahedral_complex(30, 3)
    small_seeds = (40 + np.arange(4)).astype(np.uint64)
    small_orders = np.stack([_lib.decode_order(small.atom_sources, int(s)) for s in small_seeds])
    _say("noalloc design L=300 B=16 (shared order), then L=120 B=4 (per-sequence orders, 4 chains)")
    a1 = _design(gpu_ctx, "hkbs_pmpnn_design_device_noalloc", big, 16, big_order, 1, big_seeds, 0.1)
    a2 = _design(gpu_ctx, "hkbs_pmpnn_design_device_noalloc", small, 4, small_orders, 0, small_seeds, 0.2)
    _say("device design, same inputs")
    b1 = _design(gpu_ctx, "hkbs_pmpnn_design_device", big, 16, big_order, 1, big_seeds, 0.1)
    b2 = _design(gpu_ctx, "hkbs_pmpnn_design_device", small, 4, small_orders, 0, small_seeds, 0.2)
    for got, want in ((a1, b1), (a2, b2)):
        assert np.isfinite(got[2]).all()
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)


def test_noalloc_design_refuses_oversized_request(gpu_ctx):
    lib = _lib.load()
    bb = backbone.single_chain(4000, 1)
    order = _lib.decode_order(bb.atom_sources, 1)
    d = [_dev(bb.coords), _dev(bb.atom_sources), _dev(order), _dev(np.array([1], np.uint64))]
    out = [hip.DeviceBuffer(4000 * 4), hip.DeviceBuffer(4000 * 21 * 4), hip.DeviceBuffer(4)]
    st = lib.hkbs_pmpnn_design_device_noalloc(gpu_ctx._h, d[0].ptr, d[1].ptr, None, None, None, None, 4000, 1,
                                              d[2].ptr, 1, d[3].ptr, C.c_float(0.1), 0, out[0].ptr, out[1].ptr,
                                              out[2].ptr, None)
    assert st == _lib.INVALID_ARGUMENT
    assert "128 MiB" in lib.hkbs_last_error().decode()


def _mem_free():
    free, total = C.c_size_t(), C.c_size_t()
    hip.check(hip.rt().hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
    return free.value


def test_noalloc_design_allocates_nothing_and_replays_in_a_graph(gpu_ctx):
    lib = _lib.load()
    rt = hip.rt()
    bb = backbone.single_chain(120, 5)
    L, B, T = bb.L, 8, 0.1
    order = _lib.decode_order(bb.atom_sources, 5)
    seeds = (5 + np.arange(B)).astype(np.uint64)
    c, s, od, sd = _dev(bb.coords), _dev(bb.atom_sources), _dev(order), _dev(seeds)
    outs = [hip.DeviceBuffer(B * L * 4), hip.DeviceBuffer(B * L * 21 * 4), hip.DeviceBuffer(B * 4)]

    def call(stream):
        return lib.hkbs_pmpnn_design_device_noalloc(gpu_ctx._h, c.ptr, s.ptr, None, None, None, None, L, B, od.ptr, 1,
                                                    sd.ptr, C.c_float(T), 0, outs[0].ptr, outs[1].ptr, outs[2].ptr,
                                                    stream)

    def results():
        return (_host(outs[0], (B, L), np.int32), _host(outs[1], (B, L, 21), np.float32),
                _host(outs[2], (B,), np.float32))

    def clear():
        for o in outs:
            hip.check(rt.hipMemset(o.ptr, 0xFF, C.c_size_t(o.nbytes)), "memset")

    _say("noalloc design L=120 B=8 eager (reference bits; loads every kernel)")
    _lib.check(call(None))
    hip.device_synchronize()
    want = results()
    assert np.isfinite(want[2]).all()
    _say("noalloc design: device free memory before and after a call")
    free0 = _mem_free()
    clear()
    _lib.check(call(None))
    hip.device_synchronize()
    assert _mem_free() == free0
    for g, w in zip(results(), want):
        np.testing.assert_array_equal(g, w)

    _say("noalloc design captured on a caller stream into a HIP graph")
    st = hip.Stream()
    graph, exe = C.c_void_p(), C.c_void_p()
    hip.check(rt.hipStreamBeginCapture(st.h, C.c_int(0)), "hipStreamBeginCapture")  # hipStreamCaptureModeGlobal
    rc = call(st.h)
    end = rt.hipStreamEndCapture(st.h, C.byref(graph))
    _lib.check(rc)
    hip.check(end, "hipStreamEndCapture")
    try:
        hip.check(rt.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)), "hipGraphInstantiate")
        other = backbone.single_chain(64, 9)
        oseeds = np.array([3, 4], np.uint64)
        for rep in range(3):
            clear()
            # the program's own eager work on the context's stream between replays
            gpu_ctx.design(other.coords, other.atom_sources, 2, oseeds, order_seeds=oseeds, temperature=0.2)
            _say(f"  graph replay {rep}")
            hip.check(rt.hipGraphLaunch(exe, st.h), "hipGraphLaunch")
            st.sync()
            for g, w in zip(results(), want):
                np.testing.assert_array_equal(g, w, err_msg=f"replay {rep}")
    finally:
        if exe:
            rt.hipGraphExecDestroy(exe)
        if graph:
            rt.hipGraphDestroy(graph)
        st.destroy()
