"""ctypes bindings for the CPU oracle and the reference build (test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (hikoboshi_amd) never does.

- ``Oracle``: oracle/liboracle.so, the plain-C restatement (pmpnn_oracle.c).
- ``Reference``: oracle/_ref/libhkbs_ref.so, the reference's own sources built
  by oracle/ref.mk (present only when it was built where the reference
  checkout exists; the file then travels with the tree).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libhkbs_ref.so"
V = 21
H = 128

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u8p = C.POINTER(C.c_uint8)
_f64p = C.POINTER(C.c_double)


def _p(a, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctype)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def _u8(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint8)


def k_of(L: int) -> int:
    return min(48, L)


class _TensorTable:
    def __init__(self, tensors):
        self.keep = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
        self.table = (C.POINTER(C.c_float) * len(self.keep))(*[t.ctypes.data_as(_f32p) for t in self.keep])


class Oracle:
    """The C restatement of the reference path."""

    def __init__(self, tensors, path: Path = ORACLE_SO):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        lib = C.CDLL(str(path))
        lib.pmo_model_create.restype = C.c_void_p
        lib.pmo_model_create.argtypes = [C.c_void_p]
        lib.pmo_model_destroy.argtypes = [C.c_void_p]
        lib.pmo_fast_exp_neg.restype = C.c_float
        lib.pmo_fast_exp_neg.argtypes = [C.c_float]
        lib.pmo_gelu.restype = C.c_float
        lib.pmo_gelu.argtypes = [C.c_float]
        for name in ("pmo_edge_features", "pmo_encode", "pmo_decode_order", "pmo_decode",
                     "pmo_teacher_forced_decode", "pmo_inverse_fold", "pmo_teacher_forced",
                     "pmo_algorithm_inverse_fold"):
            getattr(lib, name).restype = C.c_int
        self.lib = lib
        self._t = _TensorTable(tensors)
        self.model = C.c_void_p(lib.pmo_model_create(C.cast(self._t.table, C.c_void_p)))

    def __del__(self):
        try:
            self.lib.pmo_model_destroy(self.model)
        except Exception:
            pass

    def fast_exp_neg(self, x: float) -> float:
        return float(self.lib.pmo_fast_exp_neg(C.c_float(x)))

    def gelu(self, x: float) -> float:
        return float(self.lib.pmo_gelu(C.c_float(x)))

    def knn(self, ca, valid, K):
        ca = _f32(ca)
        valid = _u8(valid)
        L = ca.shape[0]
        idx = np.empty((L, K), np.int32)
        d2 = np.empty((L, K), np.float32)
        self.lib.pmo_knn(_p(ca, _f32p), _p(valid, _u8p), C.c_int32(L), C.c_int32(K), _p(idx, _i32p), _p(d2, _f32p))
        return idx, d2

    def edge_features(self, bb):
        L = bb.L
        K = k_of(L)
        idx = np.empty((L, K), np.int32)
        feat = np.empty((L, K, 416), np.float32)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        st = self.lib.pmo_edge_features(self.model, _p(c, _f32p), _p(s, _u8p), _p(r, _i32p), _p(ch, _i32p),
                                        C.c_int32(L), _p(idx, _i32p), _p(feat, _f32p))
        assert st == 0
        return idx, feat

    def encode(self, bb):
        L = bb.L
        K = k_of(L)
        mask = np.empty(L, np.float32)
        idx = np.empty((L, K), np.int32)
        hv = np.empty((L, H), np.float32)
        he = np.empty((L, K, H), np.float32)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        st = self.lib.pmo_encode(self.model, _p(c, _f32p), _p(s, _u8p), _p(r, _i32p), _p(ch, _i32p),
                                 C.c_int32(L), _p(mask, _f32p), _p(idx, _i32p), _p(hv, _f32p), _p(he, _f32p))
        assert st == 0
        return mask, idx, hv, he

    def decode_order(self, L, seed, chain_mask=None, residue_mask=None, input_order=None, use_input=False):
        order = np.empty(L, np.int32)
        cm, rm, io = _f32(chain_mask), _f32(residue_mask), _i32(input_order)
        st = self.lib.pmo_decode_order(_p(cm, _f32p), _p(rm, _f32p), C.c_int32(L), C.c_uint64(seed),
                                       _p(io, _i32p), C.c_int(int(use_input)), _p(order, _i32p))
        if st != 0:
            raise ValueError("invalid decoding order")
        return order

    def decode(self, enc, order, seed, temperature, greedy=False, chain_mask=None, true_tokens=None,
               forced_tokens=None):
        mask, idx, hv, he = enc
        L = hv.shape[0]
        tokens = np.empty(L, np.int32)
        lp = np.empty((L, V), np.float32)
        score = C.c_float(0)
        sampled = np.empty(L, np.int32)
        gap = np.empty(L, np.float64)
        cm, tt, ft, od = _f32(chain_mask), _i32(true_tokens), _i32(forced_tokens), _i32(order)
        st = self.lib.pmo_decode(self.model, _p(mask, _f32p), _p(idx, _i32p), _p(hv, _f32p), _p(he, _f32p),
                                 C.c_int32(L), _p(cm, _f32p), _p(tt, _i32p), _p(od, _i32p), C.c_uint64(seed),
                                 C.c_float(temperature), C.c_int(int(greedy)), _p(ft, _i32p), _p(tokens, _i32p),
                                 _p(lp, _f32p), C.byref(score), _p(sampled, _i32p), _p(gap, _f64p))
        assert st == 0
        return dict(tokens=tokens, log_probs=lp, score=score.value, sampled=sampled, cdf_gap=gap)

    def teacher_forced_decode(self, enc, tokens, order, chain_mask=None):
        mask, idx, hv, he = enc
        L = hv.shape[0]
        lp = np.empty((L, V), np.float32)
        score = C.c_float(0)
        cm, tk, od = _f32(chain_mask), _i32(tokens), _i32(order)
        st = self.lib.pmo_teacher_forced_decode(self.model, _p(mask, _f32p), _p(idx, _i32p), _p(hv, _f32p),
                                                _p(he, _f32p), C.c_int32(L), _p(cm, _f32p), _p(tk, _i32p),
                                                _p(od, _i32p), _p(lp, _f32p), C.byref(score))
        if st != 0:
            raise ValueError("invalid teacher-forced request")
        return lp, score.value

    def inverse_fold(self, bb, seed, order_seed, temperature, greedy=False, input_order=None,
                     use_input_order=False, chain_mask=None, true_tokens=None):
        L = bb.L
        tokens = np.empty(L, np.int32)
        lp = np.empty((L, V), np.float32)
        order = np.empty(L, np.int32)
        score = C.c_float(0)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        cm, io, tt = _f32(chain_mask), _i32(input_order), _i32(true_tokens)
        st = self.lib.pmo_inverse_fold(self.model, _p(c, _f32p), _p(s, _u8p), C.c_int32(L), _p(r, _i32p),
                                       _p(ch, _i32p), _p(cm, _f32p), _p(io, _i32p), _p(tt, _i32p),
                                       C.c_uint64(seed), C.c_uint64(order_seed), C.c_float(temperature),
                                       C.c_int(int(greedy)), C.c_int(int(use_input_order)), _p(tokens, _i32p),
                                       _p(lp, _f32p), _p(order, _i32p), C.byref(score))
        assert st == 0
        return dict(tokens=tokens, log_probs=lp, order=order, score=score.value)

    def teacher_forced(self, bb, tokens, input_order=None, chain_mask=None):
        L = bb.L
        lp = np.empty((L, V), np.float32)
        score = C.c_float(0)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        cm, tk, io = _f32(chain_mask), _i32(tokens), _i32(input_order)
        st = self.lib.pmo_teacher_forced(self.model, _p(c, _f32p), _p(s, _u8p), C.c_int32(L), _p(r, _i32p),
                                         _p(ch, _i32p), _p(cm, _f32p), _p(tk, _i32p), _p(io, _i32p),
                                         _p(lp, _f32p), C.byref(score))
        assert st == 0
        return lp, score.value

    def algorithm_inverse_fold(self, bb, num_seqs, seed, temperature, n_to_c=False):
        L = bb.L
        tokens = np.empty((num_seqs, L), np.int32)
        lp = np.empty((num_seqs, L, V), np.float32)
        scores = np.empty(num_seqs, np.float32)
        c, s = _f32(bb.coords), _u8(bb.atom_sources)
        st = self.lib.pmo_algorithm_inverse_fold(self.model, _p(c, _f32p), _p(s, _u8p), C.c_int32(L),
                                                 C.c_int32(num_seqs), C.c_uint64(seed), C.c_float(temperature),
                                                 C.c_int(int(n_to_c)), _p(tokens, _i32p), _p(lp, _f32p),
                                                 _p(scores, _f32p))
        assert st == 0
        return dict(tokens=tokens, log_probs=lp, scores=scores)


class Reference:
    """The reference's own sources compiled by oracle/ref.mk."""

    def __init__(self, tensors, path: Path = REF_SO):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} not built")
        lib = C.CDLL(str(path))
        lib.ref_set_weights.argtypes = [C.c_void_p]
        for name in ("ref_inverse_fold", "ref_teacher_forced", "ref_algorithm_inverse_fold",
                     "ref_algorithm_inverse_fold_ex", "ref_write_design_outputs"):
            getattr(lib, name).restype = C.c_int
        self.lib = lib
        self._t = _TensorTable(tensors)
        lib.ref_set_weights(C.cast(self._t.table, C.c_void_p))

    @staticmethod
    def available() -> bool:
        return REF_SO.exists()

    def knn(self, ca, valid, K):
        ca = _f32(ca)
        valid = _u8(valid)
        L = ca.shape[0]
        idx = np.empty((L, K), np.int32)
        d2 = np.empty((L, K), np.float32)
        self.lib.ref_knn(_p(ca, _f32p), _p(valid, _u8p), C.c_int32(L), C.c_int32(K), _p(idx, _i32p), _p(d2, _f32p))
        return idx, d2

    def inverse_fold(self, bb, seed, order_seed, temperature, greedy=False, input_order=None,
                     use_input_order=False, chain_mask=None, true_tokens=None):
        L = bb.L
        tokens = np.empty(L, np.int32)
        lp = np.empty((L, V), np.float32)
        order = np.empty(L, np.int32)
        score = C.c_float(0)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        cm, io, tt = _f32(chain_mask), _i32(input_order), _i32(true_tokens)
        st = self.lib.ref_inverse_fold(_p(c, _f32p), _p(s, _u8p), C.c_int32(L), _p(r, _i32p), _p(ch, _i32p),
                                       _p(cm, _f32p), _p(io, _i32p), _p(tt, _i32p), C.c_uint64(seed),
                                       C.c_uint64(order_seed), C.c_float(temperature), C.c_int(int(greedy)),
                                       C.c_int(int(use_input_order)), _p(tokens, _i32p), _p(lp, _f32p),
                                       _p(order, _i32p), C.byref(score))
        assert st == 0, st
        return dict(tokens=tokens, log_probs=lp, order=order, score=score.value)

    def teacher_forced(self, bb, tokens, input_order=None, chain_mask=None):
        L = bb.L
        lp = np.empty((L, V), np.float32)
        score = C.c_float(0)
        c, s, r, ch = _f32(bb.coords), _u8(bb.atom_sources), _i32(bb.residue_indices), _i32(bb.chain_labels)
        cm, tk, io = _f32(chain_mask), _i32(tokens), _i32(input_order)
        st = self.lib.ref_teacher_forced(_p(c, _f32p), _p(s, _u8p), C.c_int32(L), _p(r, _i32p), _p(ch, _i32p),
                                         _p(cm, _f32p), _p(tk, _i32p), _p(io, _i32p), _p(lp, _f32p),
                                         C.byref(score))
        assert st == 0, st
        return lp, score.value

    def algorithm_inverse_fold(self, bb, num_seqs, seed, temperature, n_to_c=False):
        L = bb.L
        tokens = np.empty((num_seqs, L), np.int32)
        lp = np.empty((num_seqs, L, V), np.float32)
        scores = np.empty(num_seqs, np.float32)
        c, s = _f32(bb.coords), _u8(bb.atom_sources)
        st = self.lib.ref_algorithm_inverse_fold(_p(c, _f32p), _p(s, _u8p), C.c_int32(L), C.c_int32(num_seqs),
                                                 C.c_uint64(seed), C.c_float(temperature), C.c_int(int(n_to_c)),
                                                 _p(tokens, _i32p), _p(lp, _f32p), _p(scores, _f32p))
        assert st == 0, st
        return dict(tokens=tokens, log_probs=lp, scores=scores)

    def algorithm_inverse_fold_ex(self, bb, num_seqs, seed, temperature, n_to_c=False, backbone_noise=0.0,
                                  residue_codes=None):
        """The reference's per-sample loop with backbone noise and native residue codes."""
        L = bb.L
        tokens = np.empty((num_seqs, L), np.int32)
        lp = np.empty((num_seqs, L, V), np.float32)
        scores = np.empty(num_seqs, np.float64)
        rec = np.empty(num_seqs, np.float64)
        rec_ok = np.empty(num_seqs, np.int32)
        c, s = _f32(bb.coords), _u8(bb.atom_sources)
        codes = None if residue_codes is None else C.create_string_buffer(residue_codes.encode(), L)
        st = self.lib.ref_algorithm_inverse_fold_ex(
            _p(c, _f32p), _p(s, _u8p), codes, C.c_int32(L), C.c_int32(num_seqs), C.c_uint64(seed),
            C.c_float(temperature), C.c_int(int(n_to_c)), C.c_float(backbone_noise), _p(tokens, _i32p),
            _p(lp, _f32p), scores.ctypes.data_as(C.c_void_p), rec.ctypes.data_as(C.c_void_p), _p(rec_ok, _i32p))
        if st != 0:
            raise ValueError(f"reference status {st}")
        return dict(tokens=tokens, log_probs=lp, scores=scores,
                    recovery=[float(r) if ok else None for r, ok in zip(rec, rec_ok)])

    def write_design_outputs(self, fasta_path, npz_path, sequences, scores, seeds, n_to_c, temperature,
                             log_probs=None):
        """The reference's FASTA / NPZ writers (cpp/io/design_fasta_writer.cpp) on plain arrays."""
        n = len(sequences)
        L = len(sequences[0]) if n else 0
        seq = C.create_string_buffer("".join(sequences).encode(), max(1, n * L))
        sc = np.ascontiguousarray(scores, np.float64)
        sd = np.ascontiguousarray(seeds, np.uint64)
        lp = None if log_probs is None else np.ascontiguousarray(log_probs, np.float32)
        st = self.lib.ref_write_design_outputs(
            (fasta_path or "").encode(), (npz_path or "").encode(), C.c_int32(n), C.c_int32(L), seq,
            sc.ctypes.data_as(C.c_void_p), sd.ctypes.data_as(C.c_void_p), C.c_int(int(n_to_c)),
            C.c_float(temperature), None if lp is None else _p(lp, _f32p))
        if st != 0:
            raise ValueError(f"reference status {st}")

    def load_structure(self, *, path=None, content=None, fmt="pdb", label="", model_index=None, model_id="",
                       chain_id="", chain_index=None, infer=True, include_modified=True):
        """The reference's structure loader (cpp/io/structure_loader.cpp:167-276): a file when ``path`` is
        given, else ``content`` parsed as ``fmt`` ("pdb" / "mmcif"). Returns (status, detail, result dict or
        None)."""
        lib = self.lib
        lib.ref_structure_load.restype = C.c_int
        lib.ref_structure_load.argtypes = [C.c_int, C.c_char_p, C.c_char_p, C.c_size_t, C.c_char_p, C.c_int, C.c_int,
                                           C.c_char_p, C.c_char_p, C.c_int, C.c_uint64, C.c_int, C.c_int,
                                           C.POINTER(C.c_void_p), C.POINTER(C.c_char_p)]
        lib.ref_structure_count.restype = C.c_size_t
        lib.ref_structure_count.argtypes = [C.c_void_p]
        lib.ref_structure_arrays.restype = C.c_size_t
        lib.ref_structure_arrays.argtypes = [C.c_void_p] + [C.c_void_p] * 7
        lib.ref_structure_text.restype = C.c_char_p
        lib.ref_structure_text.argtypes = [C.c_void_p, C.c_size_t]
        lib.ref_structure_model_index.argtypes = [C.c_void_p]
        lib.ref_structure_free.argtypes = [C.c_void_p]
        data = None if content is None else (content.encode() if isinstance(content, str) else bytes(content))
        source = 0 if path is not None else (1 if fmt == "pdb" else 2)
        h, detail = C.c_void_p(), C.c_char_p()
        st = lib.ref_structure_load(source, None if path is None else str(path).encode(), data,
                                    0 if data is None else len(data), label.encode(), int(model_index is not None),
                                    int(model_index or 0), model_id.encode(), chain_id.encode(),
                                    int(chain_index is not None), int(chain_index or 0), int(infer),
                                    int(include_modified), C.byref(h), C.byref(detail))
        msg = (detail.value or b"").decode()
        if st != 0:
            return st, msg, None
        try:
            L = int(lib.ref_structure_count(h))
            coords = np.zeros((L, 5, 3), np.float32)
            src = np.zeros((L, 5), np.uint8)
            codes = C.create_string_buffer(max(L, 1))
            numbers = np.zeros(L, np.int32)
            icodes = np.zeros(L, np.uint8)
            records = np.zeros(L, np.int64)
            breaks = np.zeros(max(L, 1), np.uint64)
            vp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
            nb = lib.ref_structure_arrays(h, vp(coords), vp(src), C.cast(codes, C.c_void_p), vp(numbers), vp(icodes),
                                          vp(records), vp(breaks))
            text = [lib.ref_structure_text(h, f).decode("utf-8", "replace") for f in range(5)]
            names = [lib.ref_structure_text(h, 5 + i).decode("utf-8", "replace") for i in range(L)]
            out = dict(coords=coords, atom_sources=src, residue_codes=codes.raw[:L].decode(), residue_numbers=numbers,
                       insertion_codes=icodes, source_record_indices=records,
                       chain_breaks=tuple(int(b) for b in breaks[:nb]), input_id=text[0], source_filename=text[1],
                       model_id=text[2], chain_id=text[3], altloc_note=text[4], residue_names=names,
                       model_index=int(lib.ref_structure_model_index(h)))
        finally:
            lib.ref_structure_free(h)
        return 0, msg, out

    def detect_structure_format(self, path, content):
        data = content.encode() if isinstance(content, str) else bytes(content)
        self.lib.ref_detect_structure_format.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        return {0: "unknown", 1: "pdb", 2: "mmcif"}[self.lib.ref_detect_structure_format(str(path).encode(), data,
                                                                                           len(data))]

    def residue_template(self):
        out = np.zeros((5, 3), np.float32)
        self.lib.ref_residue_template(out.ctypes.data_as(C.c_void_p))
        return out

    def virtual_cb(self, n, ca, c):
        a = [np.ascontiguousarray(v, np.float32) for v in (n, ca, c)]
        out = np.zeros(3, np.float32)
        self.lib.ref_virtual_cb(*[v.ctypes.data_as(C.c_void_p) for v in a], out.ctypes.data_as(C.c_void_p))
        return out
