"""The allocation-free design entry point through the C ABI.

hkbs_pmpnn_design_device_noalloc runs the kernels of hkbs_pmpnn_design_device
with its scratch in one static device array per GPU, so its outputs must be
bit-identical to that entry point's on the same inputs. Two calls in a row (the
second smaller, with per-sequence orders, chain labels and residue offsets)
check that what the first call leaves in the shared array does not leak into
the second; an oversized request is refused before any GPU work.
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
