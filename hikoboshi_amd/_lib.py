"""ctypes binding of the C ABI in include/hkbs_pmpnn.h and include/hkbs_structure.h
(libhkbs_pmpnn.so).

The product path has no fallback: if the HIP library is missing or no GPU is
visible, calls raise HkbsError.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libhkbs_pmpnn.so"

OK, INVALID_ARGUMENT, FAILED_PRECONDITION, UNAVAILABLE, UNIMPLEMENTED, INTERNAL_ERROR = range(6)
STATUS_NAMES = {
    0: "Ok", 1: "InvalidArgument", 2: "FailedPrecondition", 3: "Unavailable", 4: "Unimplemented", 5: "InternalError",
}
ORDER_RANDOM, ORDER_INPUT_PER_SEQUENCE, ORDER_INPUT_SHARED, ORDER_N_TO_C = range(4)
PRECISION_FP32, PRECISION_BF16, PRECISION_FP16, PRECISION_BF16X3 = range(4)

#: Symbols declared in include/*.h.
EXPORTS = (
    "hkbs_last_error", "hkbs_version", "hkbs_device_count", "hkbs_pmpnn_create", "hkbs_pmpnn_destroy",
    "hkbs_pmpnn_design", "hkbs_pmpnn_design_device", "hkbs_pmpnn_design_device_noalloc", "hkbs_pmpnn_score",
    "hkbs_pmpnn_decode_order",
    "hkbs_pmpnn_knn", "hkbs_pmpnn_encode", "hkbs_pmpnn_edge_features", "hkbs_pmpnn_set_timing",
    "hkbs_pmpnn_last_timing", "hkbs_pmpnn_score_batch", "hkbs_pmpnn_backbone_noise", "hkbs_pmpnn_set_precision",
    "hkbs_structure_default_options", "hkbs_structure_detect_format", "hkbs_structure_load_file",
    "hkbs_structure_load_buffer", "hkbs_structure_free", "hkbs_structure_residue_count", "hkbs_structure_coords",
    "hkbs_structure_atom_sources", "hkbs_structure_residue_codes", "hkbs_structure_model_index",
    "hkbs_structure_text", "hkbs_structure_residue_name", "hkbs_structure_residue_numbering",
    "hkbs_structure_chain_break_count", "hkbs_structure_chain_breaks", "hkbs_structure_chain_count",
    "hkbs_structure_chain_name", "hkbs_structure_chain_labels",
)
FORMAT_UNKNOWN, FORMAT_PDB, FORMAT_MMCIF = range(3)
TEXT_INPUT_ID, TEXT_SOURCE_FILENAME, TEXT_MODEL_ID, TEXT_CHAIN_ID, TEXT_ALTLOC_NOTE = range(5)


class StructureOptions(C.Structure):
    """hkbs_structure_options (include/hkbs_structure.h)."""

    _fields_ = [("has_model_index", C.c_int32), ("model_index", C.c_int32), ("model_id", C.c_char_p),
                ("chain_id", C.c_char_p), ("has_chain_index", C.c_int32), ("chain_index", C.c_uint64),
                ("infer_missing_atoms", C.c_int32), ("include_modified_residues", C.c_int32),
                ("chain_ids", C.POINTER(C.c_char_p)), ("n_chain_ids", C.c_size_t), ("all_chains", C.c_int32)]


class HkbsError(RuntimeError):
    def __init__(self, code: int, detail: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {detail}")
        self.code = code
        self.detail = detail


_vp = C.c_void_p
_i32 = C.c_int32
_sz = C.c_size_t
_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HkbsError(UNAVAILABLE, f"HIP library not built: {LIB_PATH} (run python -m hikoboshi_amd.build)")
    lib = C.CDLL(str(LIB_PATH))
    lib.hkbs_last_error.restype = C.c_char_p
    lib.hkbs_version.restype = C.c_char_p
    lib.hkbs_device_count.restype = _i32
    lib.hkbs_pmpnn_create.restype = _i32
    lib.hkbs_pmpnn_create.argtypes = [_vp, _sz, _i32, C.POINTER(_vp)]
    lib.hkbs_pmpnn_destroy.argtypes = [_vp]
    lib.hkbs_pmpnn_design.restype = _i32
    lib.hkbs_pmpnn_design.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp,
                                      C.c_float, _i32, _vp, _vp, _vp, _vp]
    lib.hkbs_pmpnn_design_device.restype = _i32
    lib.hkbs_pmpnn_design_device.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _vp,
                                             C.c_float, _i32, _vp, _vp, _vp, _vp]
    lib.hkbs_pmpnn_design_device_noalloc.restype = _i32
    lib.hkbs_pmpnn_design_device_noalloc.argtypes = lib.hkbs_pmpnn_design_device.argtypes
    lib.hkbs_pmpnn_score.restype = _i32
    lib.hkbs_pmpnn_score.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp]
    lib.hkbs_pmpnn_score_batch.restype = _i32
    lib.hkbs_pmpnn_score_batch.argtypes = [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.hkbs_pmpnn_backbone_noise.restype = _i32
    lib.hkbs_pmpnn_backbone_noise.argtypes = [_vp, _vp, _i32, C.c_float, C.c_uint64, _vp]
    lib.hkbs_pmpnn_decode_order.restype = _i32
    lib.hkbs_pmpnn_decode_order.argtypes = [_vp, _vp, _i32, C.c_uint64, _vp]
    lib.hkbs_pmpnn_knn.restype = _i32
    lib.hkbs_pmpnn_knn.argtypes = [_vp, _vp, _vp, _i32, _vp, _vp]
    lib.hkbs_pmpnn_encode.restype = _i32
    lib.hkbs_pmpnn_encode.argtypes = [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp]
    lib.hkbs_pmpnn_edge_features.restype = _i32
    lib.hkbs_pmpnn_edge_features.argtypes = [_vp, _vp, _vp, _vp, _vp, _i32, _vp]
    lib.hkbs_pmpnn_set_precision.restype = _i32
    lib.hkbs_pmpnn_set_precision.argtypes = [_vp, _i32]
    lib.hkbs_pmpnn_set_timing.restype = _i32
    lib.hkbs_pmpnn_set_timing.argtypes = [_vp, _i32]
    lib.hkbs_pmpnn_last_timing.restype = _i32
    lib.hkbs_pmpnn_last_timing.argtypes = [_vp, _vp]
    opts = C.POINTER(StructureOptions)
    lib.hkbs_structure_default_options.argtypes = [opts]
    lib.hkbs_structure_detect_format.restype = _i32
    lib.hkbs_structure_detect_format.argtypes = [C.c_char_p, C.c_char_p, _sz]
    lib.hkbs_structure_load_file.restype = _i32
    lib.hkbs_structure_load_file.argtypes = [C.c_char_p, opts, C.POINTER(_vp)]
    lib.hkbs_structure_load_buffer.restype = _i32
    lib.hkbs_structure_load_buffer.argtypes = [C.c_char_p, _sz, _i32, C.c_char_p, opts, C.POINTER(_vp)]
    lib.hkbs_structure_free.argtypes = [_vp]
    lib.hkbs_structure_residue_count.restype = _sz
    lib.hkbs_structure_residue_count.argtypes = [_vp]
    lib.hkbs_structure_coords.restype = C.POINTER(C.c_float)
    lib.hkbs_structure_coords.argtypes = [_vp]
    lib.hkbs_structure_atom_sources.restype = C.POINTER(C.c_uint8)
    lib.hkbs_structure_atom_sources.argtypes = [_vp]
    lib.hkbs_structure_residue_codes.restype = C.c_char_p
    lib.hkbs_structure_residue_codes.argtypes = [_vp]
    lib.hkbs_structure_model_index.restype = _i32
    lib.hkbs_structure_model_index.argtypes = [_vp]
    lib.hkbs_structure_text.restype = C.c_char_p
    lib.hkbs_structure_text.argtypes = [_vp, _i32]
    lib.hkbs_structure_residue_name.restype = C.c_char_p
    lib.hkbs_structure_residue_name.argtypes = [_vp, _sz]
    lib.hkbs_structure_residue_numbering.restype = _i32
    lib.hkbs_structure_residue_numbering.argtypes = [_vp, _vp, _vp, _vp]
    lib.hkbs_structure_chain_break_count.restype = _sz
    lib.hkbs_structure_chain_break_count.argtypes = [_vp]
    lib.hkbs_structure_chain_breaks.restype = C.POINTER(C.c_uint64)
    lib.hkbs_structure_chain_breaks.argtypes = [_vp]
    lib.hkbs_structure_chain_count.restype = _sz
    lib.hkbs_structure_chain_count.argtypes = [_vp]
    lib.hkbs_structure_chain_name.restype = C.c_char_p
    lib.hkbs_structure_chain_name.argtypes = [_vp, _sz]
    lib.hkbs_structure_chain_labels.restype = _i32
    lib.hkbs_structure_chain_labels.argtypes = [_vp, _vp]
    _lib = lib
    return lib


def check(code: int) -> None:
    if code != OK:
        detail = load().hkbs_last_error()
        raise HkbsError(code, detail.decode() if detail else "")


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_vp)


def f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def u8(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint8)


def u64(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint64)


def version() -> str:
    return load().hkbs_version().decode()


def device_count() -> int:
    return int(load().hkbs_device_count())


def backbone_noise(coords, atom_sources, sigma: float, seed: int) -> np.ndarray:
    """Coordinates plus the reference's per-sample Gaussian backbone noise (host)."""
    c = f32(coords)
    src = u8(atom_sources)
    out = np.empty_like(c)
    check(load().hkbs_pmpnn_backbone_noise(ptr(c), ptr(src), int(c.shape[0]), C.c_float(sigma), C.c_uint64(seed),
                                           ptr(out)))
    return out


def decode_order(atom_sources: np.ndarray, seed: int, chain_mask: np.ndarray | None = None) -> np.ndarray:
    """The reference's random decoding order (host routine of the library)."""
    src = u8(atom_sources)
    L = src.shape[0]
    order = np.empty(L, np.int32)
    cm = f32(chain_mask)
    check(load().hkbs_pmpnn_decode_order(ptr(cm), ptr(src), L, C.c_uint64(seed), ptr(order)))
    return order


class Context:
    """One weight upload on one HIP device (hkbs_pmpnn_create)."""

    def __init__(self, package: bytes, device: int = 0):
        lib = load()
        self._lib = lib
        self._h = _vp()
        buf = np.frombuffer(package, dtype=np.uint8)
        check(lib.hkbs_pmpnn_create(ptr(buf), buf.size, device, C.byref(self._h)))

    def close(self) -> None:
        if self._h:
            self._lib.hkbs_pmpnn_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def knn(self, coords, atom_sources):
        c, s = f32(coords), u8(atom_sources)
        L = c.shape[0]
        K = min(48, L)
        idx = np.empty((L, K), np.int32)
        d2 = np.empty((L, K), np.float32)
        check(self._lib.hkbs_pmpnn_knn(self._h, ptr(c), ptr(s), L, ptr(idx), ptr(d2)))
        return idx, d2

    def edge_features(self, coords, atom_sources, residue_indices=None, chain_labels=None):
        c, s, r, ch = f32(coords), u8(atom_sources), i32(residue_indices), i32(chain_labels)
        L = c.shape[0]
        K = min(48, L)
        feat = np.empty((L, K, 416), np.float32)
        check(self._lib.hkbs_pmpnn_edge_features(self._h, ptr(c), ptr(s), ptr(r), ptr(ch), L, ptr(feat)))
        return feat

    def encode(self, coords, atom_sources, residue_indices=None, chain_labels=None):
        c, s, r, ch = f32(coords), u8(atom_sources), i32(residue_indices), i32(chain_labels)
        L = c.shape[0]
        K = min(48, L)
        mask = np.empty(L, np.float32)
        idx = np.empty((L, K), np.int32)
        hv = np.empty((L, 128), np.float32)
        he = np.empty((L, K, 128), np.float32)
        check(self._lib.hkbs_pmpnn_encode(self._h, ptr(c), ptr(s), ptr(r), ptr(ch), L, ptr(mask), ptr(idx),
                                          ptr(hv), ptr(he)))
        return mask, idx, hv, he

    def design(self, coords, atom_sources, num_seqs: int, sampler_seeds, *, order_mode: int = ORDER_RANDOM,
               orders=None, order_seeds=None, temperature: float = 0.1, greedy: bool = False,
               residue_indices=None, chain_labels=None, chain_mask=None, true_tokens=None,
               want_log_probs: bool = True):
        c, s = f32(coords), u8(atom_sources)
        L = c.shape[0]
        B = int(num_seqs)
        tokens = np.empty((B, L), np.int32)
        lp = np.empty((B, L, 21), np.float32) if want_log_probs else None
        orders_out = np.empty((B, L), np.int32)
        scores = np.empty(B, np.float32)
        r, ch, cm, tt = i32(residue_indices), i32(chain_labels), f32(chain_mask), i32(true_tokens)
        od, os_, ss = i32(orders), u64(order_seeds), u64(sampler_seeds)
        check(self._lib.hkbs_pmpnn_design(self._h, ptr(c), ptr(s), ptr(r), ptr(ch), ptr(cm), ptr(tt), L, B,
                                          int(order_mode), ptr(od), ptr(os_), ptr(ss), C.c_float(temperature),
                                          int(bool(greedy)), ptr(tokens), ptr(lp), ptr(orders_out), ptr(scores)))
        return dict(tokens=tokens, log_probs=lp, orders=orders_out, scores=scores)

    def design_device(self, coords_ptr, atom_sources_ptr, L, B, orders_ptr, shared, seeds_ptr, temperature,
                      tokens_ptr, log_probs_ptr, scores_ptr, stream_ptr=None, greedy=False,
                      residue_indices_ptr=None, chain_labels_ptr=None, chain_mask_ptr=None, true_tokens_ptr=None):
        """Device-pointer variant; all *_ptr are integer device addresses."""
        check(self._lib.hkbs_pmpnn_design_device(
            self._h, coords_ptr, atom_sources_ptr, residue_indices_ptr, chain_labels_ptr, chain_mask_ptr,
            true_tokens_ptr, int(L), int(B), orders_ptr, int(shared), seeds_ptr, C.c_float(temperature),
            int(bool(greedy)), tokens_ptr, log_probs_ptr, scores_ptr, stream_ptr))

    def set_precision(self, precision: int) -> None:
        """PRECISION_FP32 (default), PRECISION_BF16, PRECISION_FP16 or PRECISION_BF16X3 for later design calls."""
        check(self._lib.hkbs_pmpnn_set_precision(self._h, int(precision)))

    def set_timing(self, enable: bool) -> None:
        check(self._lib.hkbs_pmpnn_set_timing(self._h, int(bool(enable))))

    def last_timing(self) -> tuple[float, float, float]:
        """Milliseconds of (featurise + encode, decoder precompute, decode loop) of the last design call."""
        ms = np.zeros(3, np.float32)
        check(self._lib.hkbs_pmpnn_last_timing(self._h, ptr(ms)))
        return float(ms[0]), float(ms[1]), float(ms[2])

    def score(self, coords, atom_sources, tokens, order=None, residue_indices=None, chain_labels=None,
              chain_mask=None):
        c, s, t = f32(coords), u8(atom_sources), i32(tokens)
        L = c.shape[0]
        lp = np.empty((L, 21), np.float32)
        sc = C.c_float(0)
        r, ch, cm, od = i32(residue_indices), i32(chain_labels), f32(chain_mask), i32(order)
        check(self._lib.hkbs_pmpnn_score(self._h, ptr(c), ptr(s), ptr(r), ptr(ch), ptr(cm), ptr(t), ptr(od), L,
                                         ptr(lp), C.cast(C.byref(sc), _vp)))
        return lp, sc.value

    def score_batch(self, coords, atom_sources, tokens, offsets, orders=None):
        """Teacher-forced log-probs [sum L, 21] and scores [n] of a ragged batch."""
        c, s, t = f32(coords), u8(atom_sources), i32(tokens)
        off = np.ascontiguousarray(offsets, dtype=np.int64)
        n = off.size - 1
        lp = np.empty((int(off[-1]), 21), np.float32)
        sc = np.empty(n, np.float32)
        od = i32(orders)
        check(self._lib.hkbs_pmpnn_score_batch(self._h, n, ptr(off), ptr(c), ptr(s), ptr(t), ptr(od), ptr(lp),
                                               ptr(sc)))
        return lp, sc
