#!/usr/bin/env python3
"""Batched ProteinMPNN v_48_020 design on one MI355X.

Headline: one step = one design of B = 64 sequences on one synthetic L = 300
backbone with the inputs resident in HBM: featurise + encode + 300
autoregressive decode steps + the copy of tokens, log-probs and scores into
pinned host memory. value = B * L / step time (sampled residues/s). Every
timed step checks that all scores are finite: a decode team that failed to
assemble leaves a NaN score, so a failed design is never counted.

The JSON line also carries
  us_per_decode_step  decode-kernel time / L (HIP events on the stream the kernels run on);
  roofline            the decode kernel (the dominant kernel) against HBM bandwidth:
                      achieved = algorithmic bytes per launch / kernel time, the compulsory
                      bytes of one decode being 4 [B (3 H E_bw + L (2H + V + 1)) + L (2K + 1) H
                      + W_dec] (E_bw = kNN edges to earlier positions); traffic = HBM bytes per
                      launch from the committed rocprofv3 counters; the FLOP the launch
                      executes against the VALU fp32 and MFMA fp16 peaks; and l2_stream, the
                      bytes its L1 caches request from L2 (committed counters) over the kernel
                      time against the L2-to-L1 peak (the decoder weights are streamed from L2
                      by every workgroup in every dependency pass);
  encoder             featurise + encode against the fp32 peak;
  cpu_baseline        the reference's own scalar code (oracle/_ref) on a bounded sample of the
                      same workload, timed on this host's cores before the GPU is touched;
  configs             the other workloads: L = 120 x 8 with per-sequence random orders, the
                      4 x 256 complex x 256 sequences, the 4,096-protein teacher-forced ragged
                      batch and L = 4,000 x 32 in split bf16 (every decoder product on the bf16
                      MFMA with both operands as two bf16 terms; plain bf16 and fp32 timed beside
                      it), each with its time, throughput, a spot check against the CPU reference
                      and a CPU baseline of its own.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hikoboshi_amd import backbone  # noqa: E402  (numpy only; no GPU)

METRIC = "sampled residues/sec at L=300×64 seqs; µs per decode step"
F_RES = 29_103_360        # FLOP per sampled residue, reference arithmetic at K=48
# FLOP per sampled residue the restructured decode loop executes, split by unit: per message layer
# the W2 product over the 48 message rows (fp32 mode: on the fp16 MFMA as three products of split
# operands, hi.hi + hi.lo + lo.hi; bf16 mode: one bf16 product) and on the VALU the row sums
# A + E1 + R|Q and the column sums; on every layer W3 on the summed rows, W_in and W_out; the fused
# next-layer [W1d | W1a] of layers 0 and 1 and the logits. In fp32 mode layer 0's message rows come
# from the precomputed table (the decode then only sums 48 rows of it), so two layers are message layers.
F_W2_LAYER = 2 * 48 * 128 * 128
F_MSG_VALU_LAYER = 2 * 48 * 128 + 48 * 128
F_LOGITS = 2 * 128 * 21
F_LAYER_PRODUCTS = 3 * (2 * 128 * 128 + 2 * 2 * 128 * 512) + 2 * (2 * 128 * 256)  # W3, W_in, W_out, next [W1d | W1a]
F_VALU_REST = F_LAYER_PRODUCTS + F_LOGITS
# MFMA products per product of the 16-bit modes: bf16 / fp16 multiply the two halves of the split
# activations by one 16-bit weight; split bf16 takes hi.hi + hi.lo + lo.hi. W2's message rows are one
# bf16 / fp16 operand in those modes, two bf16 terms in split bf16.
SPLIT_PRODUCTS = {"bf16": (1, 2), "fp16": (1, 2), "bf16x3": (3, 3)}  # (W2, layer products)
PRECISION_CODES = {"fp32": 0, "bf16": 1, "fp16": 2, "bf16x3": 3}
L0_TABLE_MAX_BYTES = 4 << 30  # the library's limit for the layer-0 table (22 rows of 128 floats per slot)
W_DEC = 698_133           # decoder + W_out + W_s floats
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 (vector and matrix)
PEAK_FP16_TFLOPS = 2500.0 # MI355X dense fp16 / bf16 MFMA
PEAK_HBM_GBPS = 8000.0    # MI355X HBM3E
# L2 to L1 (the port the decode streams its weights through): 16 channels x 128 bytes a clock per XCD (the
# CDNA3 L2 design), 8 XCDs, 2.4 GHz peak engine clock; 64 bytes a clock for each of the 256 CUs.
PEAK_L2_GBPS = 16 * 128 * 8 * 2.4
H, V = 128, 21
C4_CPU_PROTEINS = 32      # proteins of the ragged batch the CPU baseline scores


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--L", type=int, default=300)
    p.add_argument("--num-seqs", type=int, default=64)
    p.add_argument("--temperature", type=float, default=0.1)
    p.add_argument("--seed", type=int, default=7)
    p.add_argument("--precision", choices=("fp32", "bf16", "bf16x3"), default="fp32",
                   help="design arithmetic of the headline workload (bf16: bf16 decoder; bf16x3: split bf16 "
                        "decoder, both operands of every product as two bf16 terms)")
    p.add_argument("--complex", action="store_true",
                   help="the main workload is the tetrahedral complex of 4 chains of --L residues (with --num-seqs "
                        "256 --temperature 0.2 and --L 256: the 4 x 256 configuration)")
    p.add_argument("--workers", type=int, default=0, help="CPU worker processes (default: min(16, host CPUs))")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--no-configs", action="store_true", help="headline workload only")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="only run a device-to-device copy of MIB MiB (HBM-counter calibration) and exit")
    p.add_argument("--score-batch", type=int, default=0, metavar="N",
                   help="only time teacher-forced scoring of a ragged batch of N synthetic proteins "
                        "(L ~ U[50, 500], native tokens) from host buffers")
    return p.parse_args()


# ------------------------------------------------------------------ inputs --

def workloads(args):
    """Synthetic inputs of every workload, built on the host before the CPU workers fork."""
    import oracle
    from hikoboshi_amd import weights

    seed = args.seed
    orc = oracle.Oracle(weights.load_tensors())

    def shared_order(bb):
        valid = (bb.atom_sources[:, :4] != 0).all(1).astype(np.float32)
        return orc.decode_order(bb.L, seed, residue_mask=valid)

    L, B = args.L, args.num_seqs
    bb = backbone.tetrahedral_complex(L, seed) if args.complex else backbone.single_chain(L, seed)
    suffix = "" if args.precision == "fp32" else "_" + args.precision
    name = f"complex_4x{L}_B{B}{suffix}" if args.complex else f"design_L{L}_B{B}{suffix}"
    W = {"C2": dict(name=name, bb=bb, B=B, T=args.temperature, order=shared_order(bb),
                    seeds=(seed + np.arange(B)).astype(np.uint64), precision=args.precision,
                    cpu_seqs=list(range(min(B, 16))))}
    if not args.no_configs:
        c1 = backbone.single_chain(120, seed)
        W["C1"] = dict(name="design_L120_B8", bb=c1, B=8, T=0.1, order=None,
                       seeds=(seed + np.arange(8)).astype(np.uint64), precision="fp32", cpu_seqs=list(range(8)))
        cx = backbone.tetrahedral_complex(256, seed)
        W["C3"] = dict(name="complex_4x256_B256", bb=cx, B=256, T=0.2, order=shared_order(cx),
                       seeds=(seed + np.arange(256)).astype(np.uint64), precision="fp32",
                       cpu_seqs=[int(b) for b in np.linspace(0, 255, 16).round()])
        c5 = backbone.single_chain(4000, seed)
        W["C5"] = dict(name="design_L4000_B32_bf16x3", bb=c5, B=32, T=0.1, order=shared_order(c5),
                       seeds=(seed + np.arange(32)).astype(np.uint64), precision="bf16x3", cpu_seqs=[0])
        coords, src, tok, off = backbone.ragged_batch(4096, seed)
        pick = np.sort(np.random.default_rng(seed).choice(4096, C4_CPU_PROTEINS, replace=False))
        W["C4"] = dict(name="score_ragged4096", batch=(coords, src, tok, off), cpu_proteins=[int(i) for i in pick])
    return W


# --------------------------------------------------------------- CPU leg --

_W = {}      # workloads, inherited by the forked workers
_IMPL = None  # per worker: the reference build (or the C restatement when it is absent)


def _init_worker():
    global _IMPL
    import oracle
    from hikoboshi_amd import weights

    tensors = weights.load_tensors()
    _IMPL = (oracle.Reference(tensors), "reference") if oracle.Reference.available() else \
        (oracle.Oracle(tensors), "port")


def _cpu_task(task):
    """One single-threaded reference call: a design module call for one sequence (it featurises and
    encodes the backbone again, as the reference's per-sample loop does) or the teacher-forced
    forward of one protein. Returns the outputs and the call's own seconds."""
    cfg, i = task
    impl, kind = _IMPL
    w = _W[cfg]
    if cfg == "C4":
        coords, src, tok, off = w["batch"]
        sl = slice(int(off[i]), int(off[i + 1]))
        t0 = time.perf_counter()
        lp, _ = impl.teacher_forced(backbone.Backbone(coords[sl], src[sl]), tok[sl])
        return cfg, i, None, lp, time.perf_counter() - t0, kind
    seed = int(w["seeds"][i])
    t0 = time.perf_counter()
    o = impl.inverse_fold(w["bb"], seed=seed, order_seed=seed, temperature=w["T"], input_order=w["order"],
                          use_input_order=w["order"] is not None)
    return cfg, i, o["tokens"], o["log_probs"], time.perf_counter() - t0, kind


def _task_cost(task):
    cfg, i = task
    if cfg == "C4":
        off = _W["C4"]["batch"][3]
        return int(off[i + 1] - off[i])
    return _W[cfg]["bb"].L


def host_cpu():
    model = ""
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def cpu_leg(workers):
    """Every CPU task of every workload in one pool of forked single-threaded workers, longest first.
    Each task times its own reference call, so worker start-up and weight loading are excluded."""
    import multiprocessing as mp

    tasks = []
    for cfg, w in _W.items():
        ids = w["cpu_proteins"] if cfg == "C4" else w["cpu_seqs"]
        tasks += [(cfg, i) for i in ids]
    tasks.sort(key=_task_cost, reverse=True)
    t0 = time.perf_counter()
    with mp.get_context("fork").Pool(workers, initializer=_init_worker) as pool:
        res = list(pool.imap_unordered(_cpu_task, tasks, chunksize=1))
    wall = time.perf_counter() - t0
    out = {}
    for cfg, i, tok, lp, dt, kind in res:
        out.setdefault(cfg, {"kind": kind, "outputs": {}, "seconds": 0.0})
        out[cfg]["outputs"][i] = (tok, lp)
        out[cfg]["seconds"] += dt
    return out, wall


def cpu_summary(cfg, got, workers, model, wall):
    """Residues per second of the reference on `workers` cores: each task's own time under the
    all-core load of the pool, cores x residues / (sum of task seconds)."""
    w = _W[cfg]
    if cfg == "C4":
        off = w["batch"][3]
        residues = int(sum(off[i + 1] - off[i] for i in got["outputs"]))
        what = (f"teacher-forced forward of {len(got['outputs'])} randomly chosen proteins of the batch "
                f"({residues} residues), one call per protein")
    else:
        residues = w["bb"].L * len(got["outputs"])
        ids = sorted(got["outputs"])
        what = (f"{len(ids)} of the {w['B']} sequences (indices {ids[0]}..{ids[-1]}), one design module call "
                f"per sequence (featurise + encode + decode, re-encoding per sequence as the reference's "
                f"per-sample loop does)")
    single = residues / got["seconds"]
    return {
        "value": round(single * workers, 2), "unit": "residues/s", "cores": workers, "kind": got["kind"],
        "sample": f"{what}, spread over {workers} forked single-threaded worker processes; value = cores x "
                  f"residues / sum of per-call seconds (start-up and weight loading excluded); the pool ran "
                  f"{wall:.1f} s for all workloads",
        "single_core_value": round(single, 3), "cpu_model": model, "seconds": round(got["seconds"], 2),
    }


def spot_check(got, tokens, log_probs):
    """Reference outputs against the GPU's for the sequences the CPU leg ran."""
    same, worst = 0, 0.0
    for b, (tok, lp) in got["outputs"].items():
        if np.array_equal(tok, tokens[b]):
            same += 1
            worst = max(worst, float(np.abs(lp - log_probs[b]).max()))
    return {"tokens_identical": same, "of": len(got["outputs"]), "max_abs_dlogp": worst if same else None}


# --------------------------------------------------------------- GPU leg --

class DeviceDesign:
    """One workload's device-resident inputs and outputs; step() = one design call on device
    buffers, the copy of its outputs to pinned host memory, a wait for the stream and a check
    that every score is finite."""

    def __init__(self, ctx, w, order):
        from hikoboshi_amd import hip

        bb, B, L = w["bb"], w["B"], w["bb"].L
        self.ctx, self.L, self.B, self.T, self.hip = ctx, L, B, w["T"], hip
        self.d = {k: hip.DeviceBuffer.from_array(v) for k, v in
                  (("coords", bb.coords), ("src", bb.atom_sources), ("order", order), ("seeds", w["seeds"]))}
        for k, v in (("resid", bb.residue_indices), ("chain", bb.chain_labels)):
            self.d[k] = hip.DeviceBuffer.from_array(v) if v is not None else None
        self.d["tokens"] = hip.DeviceBuffer(B * L * 4)
        self.d["lp"] = hip.DeviceBuffer(B * L * V * 4)
        self.d["scores"] = hip.DeviceBuffer(B * 4)
        self.h_tokens = hip.PinnedBuffer((B, L), np.int32)
        self.h_lp = hip.PinnedBuffer((B, L, V), np.float32)
        self.h_scores = hip.PinnedBuffer((B,), np.float32)
        self.stream = hip.Stream()

    def step(self):
        d, hip = self.d, self.hip
        self.ctx.design_device(d["coords"].addr, d["src"].addr, self.L, self.B, d["order"].addr, 1,
                               d["seeds"].addr, self.T, d["tokens"].addr, d["lp"].addr, d["scores"].addr,
                               stream_ptr=self.stream.h.value,
                               residue_indices_ptr=d["resid"].addr if d["resid"] else None,
                               chain_labels_ptr=d["chain"].addr if d["chain"] else None)
        hip.memcpy_d2h_async(self.h_tokens, d["tokens"], self.B * self.L * 4, self.stream)
        hip.memcpy_d2h_async(self.h_lp, d["lp"], self.B * self.L * V * 4, self.stream)
        hip.memcpy_d2h_async(self.h_scores, d["scores"], self.B * 4, self.stream)
        self.stream.sync()
        if not np.isfinite(self.h_scores.array).all():
            raise RuntimeError("a design returned a non-finite score (a decode team failed to assemble)")

    def run(self, steps, warmup):
        """ms per step over `steps` timed steps and the mean phase times (featurise + encode,
        decoder precompute, decode kernel) of those steps."""
        self.ctx.set_timing(True)
        for _ in range(warmup):
            self.step()
        self.hip.device_synchronize()
        phases = []
        t0 = time.perf_counter()
        for _ in range(steps):
            self.step()
            phases.append(self.ctx.last_timing())
        self.hip.device_synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        self.ctx.set_timing(False)
        return ms, np.mean(np.array(phases), axis=0)


def measured_traffic(workload: str):
    """HBM bytes per decode_kernel launch from the committed rocprofv3 summary, if it covers this workload."""
    path = os.path.join(ROOT, "profiles", f"decode_kernel_{workload}.md")
    key = f"decode_kernel HBM bytes per launch ({workload}):"
    try:
        with open(path, encoding="utf-8") as f:
            for line in f:
                if line.startswith(key):
                    return int(line.split(":")[1].strip()), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def measured_l2_reads(workload: str):
    """decode_kernel's L1-to-L2 read bytes per launch from the committed rocprofv3 summary, if it covers this
    workload."""
    path = os.path.join(ROOT, "profiles", f"decode_kernel_{workload}.md")
    key = f"decode_kernel L1-to-L2 read bytes per launch ({workload}):"
    try:
        with open(path, encoding="utf-8") as f:
            for line in f:
                if line.startswith(key):
                    return int(line.split(":")[1].strip()), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def l0_table_used(precision: str, L: int) -> bool:
    """Whether the library builds the layer-0 message table for this request (fp32 and split bf16)."""
    K = min(48, L)
    return precision in ("fp32", "bf16x3") and os.environ.get("HKBS_DECODE_L0TABLE") != "off" and \
        L * K * 22 * 128 * 4 <= L0_TABLE_MAX_BYTES


def decode_roofline(ctx, w, order, decode_ms, precision=None, name=None):
    """The decode kernel against HBM bandwidth (algorithmic bytes) and its executed FLOP against the
    VALU fp32 and MFMA peaks."""
    bb, B, L = w["bb"], w["B"], w["bb"].L
    K = min(48, L)
    prec = precision or w["precision"]
    table = l0_table_used(prec, L)
    msg_layers = 2 if table else 3
    if prec == "fp32":  # W2 on the fp16 MFMA (split operands), the layer products on the VALU
        f_valu = msg_layers * F_MSG_VALU_LAYER + (48 * 128 if table else 0) + F_VALU_REST
        f_mfma = 3 * msg_layers * F_W2_LAYER
        mfma_key = "mfma_fp16"
        mfma_note = (f"W2 of {msg_layers} layers as three fp16 products of split operands (hi.hi + hi.lo + lo.hi)"
                     + ("; layer 0's rows come from the layer-0 table kernel, outside this launch" if table else ""))
    else:  # W2 and the layer products on the MFMA
        w2x, lpx = SPLIT_PRODUCTS[prec]
        f_valu = msg_layers * F_MSG_VALU_LAYER + (48 * 128 if table else 0) + F_LOGITS
        f_mfma = w2x * msg_layers * F_W2_LAYER + lpx * F_LAYER_PRODUCTS
        mfma_key = "mfma_fp16" if prec == "fp16" else "mfma_bf16"
        mfma_note = (f"W2 of {'layers 1 and 2' if table else 'all three layers'} as {w2x} and W3, W_in, W_out and "
                     f"the fused next-layer product as {lpx} {'fp16' if prec == 'fp16' else 'bf16'} products each, "
                     "useful rows only (members of a pass fill rows of the 16-row tiles)"
                     + ("; layer 0's rows come from the layer-0 table kernel, outside this launch" if table else ""))
    idx, _ = ctx.knn(bb.coords, bb.atom_sources)
    pos = np.empty(L, np.int64)
    pos[order] = np.arange(L)
    e_bw = int((pos[idx] < pos[:, None]).sum())
    launch_bytes = 4.0 * (B * (3 * H * e_bw + L * (2 * H + V + 1)) + L * (2 * K + 1) * H + W_DEC)
    t = decode_ms * 1e-3
    achieved = launch_bytes / t / 1e9
    traffic, traffic_src = measured_traffic(name or w["name"])
    l2_bytes, l2_src = measured_l2_reads(name or w["name"])
    valu = B * L * f_valu / t / 1e12
    mfma = B * L * f_mfma / t / 1e12
    return {
        "kernel": "decode_kernel",
        "bound": "hbm",
        "achieved": round(achieved, 2),
        "peak": PEAK_HBM_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBPS, 5),
        "traffic": traffic,
        "kernel_ms": round(decode_ms, 4),
        "algorithmic_bytes": int(launch_bytes),
        "algorithmic_units": (f"4 [B (3 H E_bw + L (2H + V + 1)) + L (2K + 1) H + W_dec] bytes per launch, "
                              f"B={B} L={L} K={K} E_bw={e_bw} W_dec={W_DEC}"),
        "traffic_source": (f"{traffic_src}: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-kernel "
                           "calibrated), bytes per launch") if traffic else None,
        "executed": {
            "valu_fp32": {"flop_per_residue": f_valu, "achieved_tflops": round(valu, 3), "peak": PEAK_FP32_TFLOPS,
                          "frac": round(valu / PEAK_FP32_TFLOPS, 4)},
            mfma_key: {"flop_per_residue": f_mfma, "achieved_tflops": round(mfma, 3), "peak": PEAK_FP16_TFLOPS,
                       "frac": round(mfma / PEAK_FP16_TFLOPS, 4), "note": mfma_note},
            "reference_flop_per_residue": F_RES,
        },
        # every workgroup streams the decoder weights from L2 in every dependency pass: the bytes its L1s
        # request from L2 (committed counters of the same workload) over this launch's time
        "l2_stream": None if not l2_bytes else {
            "bytes": l2_bytes, "achieved": round(l2_bytes / t / 1e9, 1), "peak": round(PEAK_L2_GBPS, 1), "unit": "GB/s",
            "frac": round(l2_bytes / t / 1e9 / PEAK_L2_GBPS, 4),
            "source": f"{l2_src}: rocprofv3 TCP_TCC_READ_REQ_sum x 128 bytes, per launch"},
        "limiter": ("latency: neither HBM nor the arithmetic units are near their peaks; the SQ counters in "
                    "profiles/ show waves waiting most of their cycles on L2 weight streaming and barriers"),
    }


def score_batch_bench(args) -> int:
    """Teacher-forced log-probs of a ragged batch (hkbs_pmpnn_score_batch): one step = one call on the
    whole batch, from host buffers to host buffers (the call is synchronous, PCIe included)."""
    from hikoboshi_amd import _lib, weights

    coords, src, tokens, offsets = backbone.ragged_batch(args.score_batch, args.seed)
    ctx = _lib.Context(weights.read_package_bytes())
    for _ in range(args.warmup):
        ctx.score_batch(coords, src, tokens, offsets)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        _, sc = ctx.score_batch(coords, src, tokens, offsets)
    dt = (time.perf_counter() - t0) / args.steps
    if not np.isfinite(sc).all():
        raise RuntimeError("non-finite teacher-forced score")
    n_res = int(offsets[-1])
    print(json.dumps({
        "metric": "teacher-forced residues/sec, ragged batch", "value": round(n_res / dt, 1), "unit": "residues/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"score_ragged{args.score_batch}", "proteins": args.score_batch, "residues": n_res,
                   "L_range": [50, 500], "seed": args.seed, "inputs": "host buffers (PCIe included)"}}), flush=True)
    return 0


def calibrate_copy(mib: int) -> int:
    """One D2D copy of known size: reference point for FETCH_SIZE / WRITE_SIZE counters."""
    from hikoboshi_amd import hip

    n = mib << 20
    src, dst = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
    for _ in range(3):
        hip.check(hip.rt().hipMemcpy(dst.ptr, src.ptr, hip.C.c_size_t(n), hip.D2D), "D2D")
    hip.device_synchronize()
    print(json.dumps({"calibration_copy_bytes": n, "copies": 3}), flush=True)
    return 0


def trajectory_deviation(ctx, w, order, run, n):
    """max |d log p| of the last run's first n sequences against the fp32 path on the same trajectory:
    fp32 teacher-forced log-probs of the run's tokens and order, rescaled to the run's T (contract 2e-2)."""
    worst = 0.0
    bb = w["bb"]
    for b in range(n):
        tok = run.h_tokens.array[b].copy()
        lp1, _ = ctx.score(bb.coords, bb.atom_sources, tok, order=order)
        z = lp1.astype(np.float64) / w["T"]
        z -= z.max(1, keepdims=True)
        ref = z - np.log(np.exp(z).sum(1, keepdims=True))
        worst = max(worst, float(np.abs(run.h_lp.array[b] - ref).max()))
    return {"max_abs_dlogp": round(worst, 6), "sequences": n, "contract": 2e-2,
            "note": "fp32 teacher-forced log-probs of the run's tokens and order, at T"}


def run_configs(ctx, cpu, workers, model, wall, steps, warmup):
    """C1, C3, C4 and C5 on the GPU, each with its CPU baseline and spot check."""
    from hikoboshi_amd import _lib

    out = {}
    # C1: host buffers through hkbs_pmpnn_design, a random order per sequence (seed 7 + i for order and
    # sampler, the reference's per-sample loop), host order generation and PCIe included.
    w = _W["C1"]
    bb = w["bb"]

    def c1():
        r = ctx.design(bb.coords, bb.atom_sources, w["B"], w["seeds"], order_seeds=w["seeds"], temperature=w["T"])
        if not np.isfinite(r["scores"]).all():
            raise RuntimeError("non-finite score")
        return r

    for _ in range(warmup):
        c1()
    t0 = time.perf_counter()
    for _ in range(steps):
        r = c1()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    out["C1"] = {"workload": w["name"], "L": bb.L, "num_seqs": w["B"], "temperature": w["T"],
                 "decode_order": "random per sequence (seed 7+i, order and sampler)",
                 "inputs": "host buffers (hkbs_pmpnn_design; host order generation and PCIe included)",
                 "ms": round(ms, 4), "value": round(w["B"] * bb.L / (ms * 1e-3), 1), "unit": "residues/s"}
    if "C1" in cpu:
        out["C1"]["parity_spot_check"] = spot_check(cpu["C1"], r["tokens"], r["log_probs"])
        out["C1"]["cpu_baseline"] = cpu_summary("C1", cpu["C1"], workers, model, wall)

    # C3 and C5: device-resident inputs, outputs copied to pinned host memory (as the headline).
    for cfg in ("C3", "C5"):
        w = _W[cfg]
        order = _lib.decode_order(w["bb"].atom_sources, int(w["seeds"][0]))
        if not np.array_equal(order, w["order"]):
            raise RuntimeError(f"{cfg}: decode order differs between the library and the oracle")
        run = DeviceDesign(ctx, w, order)
        res = {"workload": w["name"], "L": w["bb"].L, "num_seqs": w["B"], "temperature": w["T"],
               "decode_order": "shared random permutation (reference routine, seed 7)",
               "inputs": "device buffers, outputs copied to pinned host memory"}
        if cfg == "C5":
            # fp32 first (the tolerance reference and the CPU spot check), then plain bf16 (kept beside
            # the result: it misses the contract), then the configuration's mode, split bf16.
            ms32, ph32 = run.run(steps, warmup)
            fp32_tokens, fp32_lp = run.h_tokens.array.copy(), run.h_lp.array.copy()
            res["fp32"] = {"ms": round(ms32, 4), "value": round(w["B"] * w["bb"].L / (ms32 * 1e-3), 1),
                           "decode_ms": round(float(ph32[2]), 4)}
            ctx.set_precision(_lib.PRECISION_BF16)
            try:
                msb, phb = run.run(steps, warmup)
            finally:
                ctx.set_precision(_lib.PRECISION_FP32)
            res["plain_bf16"] = {
                "mode": "HKBS_PRECISION_BF16: bf16 weights, bf16 message rows into W2, fp16 E1/Q/R rows",
                "ms": round(msb, 4), "value": round(w["B"] * w["bb"].L / (msb * 1e-3), 1),
                "decode_ms": round(float(phb[2]), 4),
                "bf16_vs_fp32": trajectory_deviation(ctx, w, order, run, 2)}
            ctx.set_precision(PRECISION_CODES[w["precision"]])
        try:
            ms, ph = run.run(steps, warmup)
        finally:
            ctx.set_precision(_lib.PRECISION_FP32)
        res.update({"dtype": "bf16" if cfg == "C5" else "f32", "ms": round(ms, 4),
                    "value": round(w["B"] * w["bb"].L / (ms * 1e-3), 1), "unit": "residues/s",
                    "phase_ms": {"featurise_encode": round(float(ph[0]), 4),
                                 "decoder_precompute": round(float(ph[1]), 4), "decode_loop": round(float(ph[2]), 4)},
                    "us_per_decode_step": round(float(ph[2]) * 1e3 / w["bb"].L, 3),
                    "roofline": decode_roofline(ctx, w, order, float(ph[2]))})
        if cfg == "C5":
            res["mode"] = ("HKBS_PRECISION_BF16X3 (split bf16): every decoder product on the bf16 MFMA with "
                           "weights and inputs each as two bf16 terms (hi + lo), three MFMAs per product, fp32 "
                           "accumulation, GELU, LayerNorm and softmax; E1/Q/R rows fp32; encoder on the fp16 "
                           "MFMA with split operands")
            res["bf16_vs_fp32"] = trajectory_deviation(ctx, w, order, run, w["B"])
            tokens, lps = fp32_tokens, fp32_lp
        else:
            tokens, lps = run.h_tokens.array, run.h_lp.array
        if cfg in cpu:
            res["parity_spot_check"] = spot_check(cpu[cfg], tokens, lps)
            if cfg == "C5":
                res["parity_spot_check"]["against"] = "the fp32 run"
            res["cpu_baseline"] = cpu_summary(cfg, cpu[cfg], workers, model, wall)
        out[cfg] = res

    # C4: teacher-forced scoring of the ragged batch from host buffers (synchronous, PCIe included).
    w = _W["C4"]
    coords, src, tok, off = w["batch"]
    for _ in range(max(1, warmup // 2)):
        ctx.score_batch(coords, src, tok, off)
    n4 = max(1, min(3, steps))
    t0 = time.perf_counter()
    for _ in range(n4):
        lp, sc = ctx.score_batch(coords, src, tok, off)
    ms = (time.perf_counter() - t0) * 1e3 / n4
    if not np.isfinite(sc).all():
        raise RuntimeError("non-finite teacher-forced score")
    res = {"workload": w["name"], "proteins": 4096, "residues": int(off[-1]), "L_range": [50, 500],
           "decode_order": "n_to_c", "inputs": "host buffers (hkbs_pmpnn_score_batch; PCIe included)",
           "ms": round(ms, 3), "value": round(int(off[-1]) / (ms * 1e-3), 1), "unit": "residues/s"}
    if "C4" in cpu:
        worst = max(float(np.abs(lp[off[i]:off[i + 1]] - olp).max()) for i, (_, olp) in cpu["C4"]["outputs"].items())
        res["parity_spot_check"] = {"proteins": len(cpu["C4"]["outputs"]), "max_abs_dlogp": worst}
        res["cpu_baseline"] = cpu_summary("C4", cpu["C4"], workers, model, wall)
    out["C4"] = res
    return out


def main() -> int:
    args = parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (the path shards by "
                                   "sequences across GPUs, which this benchmark does not launch)"}))
        return 2
    if args.score_batch:
        return score_batch_bench(args)

    _W.update(workloads(args))
    model, ncpu, usable = host_cpu()
    workers = args.workers or max(1, min(16, usable))
    cpu, wall = {}, 0.0
    if not args.no_cpu:
        # The CPU leg runs first, in forked workers, while this process has not touched the GPU.
        cpu, wall = cpu_leg(workers)

    from hikoboshi_amd import _lib, weights

    w = _W["C2"]
    bb, L, B, T = w["bb"], w["bb"].L, w["B"], w["T"]
    K = min(48, L)
    order = _lib.decode_order(bb.atom_sources, args.seed)
    if not np.array_equal(order, w["order"]):
        raise RuntimeError("decode order differs between the library and the oracle")
    ctx = _lib.Context(weights.read_package_bytes(), device=0)
    if args.precision != "fp32":
        ctx.set_precision(PRECISION_CODES[args.precision])
    run = DeviceDesign(ctx, w, order)
    ms_per_step, ph = run.run(args.steps, args.warmup)
    decode_ms = float(ph[2])
    f_enc = L * K * 128 * 8768 + 786432 * L  # featurise + encode FLOP per backbone
    result = {
        "metric": METRIC,
        "value": round(B * L / (ms_per_step * 1e-3), 1),
        "unit": "residues/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.precision == "fp32" else "bf16" if args.precision.startswith("bf16") else "f16",
        "data": "synthetic",
        "config": {
            "workload": w["name"],
            "L": L, "num_seqs": B, "k_neighbors": K, "temperature": T,
            "backbone": (f"4 NeRF chains of {args.L} residues on a tetrahedron, 25 A apart, seed {args.seed}"
                         if args.complex else
                         f"NeRF ideal-geometry single chain, helix/strand segments, seed {args.seed}"),
            "decode_order": f"shared random permutation (reference routine, seed {args.seed})",
            "sampler_seeds": f"{args.seed}+b (splitmix64 counter streams)",
            "weights": "ProteinMPNN v_48_020 (bundled package)",
            "step": "device-resident inputs -> designs copied to pinned host memory (D2H included)",
        },
        "us_per_decode_step": round(decode_ms * 1e3 / L, 3),
        "phase_ms": {"featurise_encode": round(float(ph[0]), 4), "decoder_precompute": round(float(ph[1]), 4),
                     "decode_loop": round(decode_ms, 4)},
        "roofline": decode_roofline(ctx, w, order, decode_ms),
        "encoder": {
            "flop": f_enc,
            "ms": round(float(ph[0]), 4),
            "achieved": round(f_enc / (float(ph[0]) * 1e-3) / 1e12, 3),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(f_enc / (float(ph[0]) * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4),
            "note": ("featurise + encode, F_enc = S*128*8768 + 786432*L FLOP per backbone; in fp32 the "
                     "encoder keeps the reference's rounding sequence (each product rounded once on the "
                     "fp32 MFMA with a zero addend, then one VALU add per product in k order) and in the "
                     "16-bit modes runs on the fp16 MFMA"),
        },
    }
    if "C2" in cpu:
        cb = cpu_summary("C2", cpu["C2"], workers, model, wall)
        cb["host_cpus"] = {"nproc": ncpu, "usable": usable}
        cb["parity_spot_check"] = spot_check(cpu["C2"], run.h_tokens.array, run.h_lp.array)
        result["cpu_baseline"] = cb
    if not args.no_configs:
        result["configs"] = run_configs(ctx, cpu, workers, model, wall, min(args.steps, 5), min(args.warmup, 2))
    ctx.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
