"""Benchmark of the MaxSim hot path on one MI355X.

Headline workload (configuration C5, the largest contrastive batch):
one contrastive training step -- score_contrastive_train over Nq=Nb=512
queries/documents (Lq=32, Ld ~ U[128, 1024], dim=128, bf16, L2-normalised
Gaussian embeddings, 1% duplicated document tokens), cross-entropy over the
diagonal, backward to dQ and dD.  Inputs are resident in HBM before timing.

Printed as ONE JSON line.  ``value`` is the step throughput in TFLOP/s
(F = 2*D*Nq*Lq*T_d forward flops per step / step time); ``ms_per_step`` is the
user-level step time (including the API's offset validation).
``extra.c5.fused_ce_step_ms`` is the same step through the fused loss
(score_contrastive_cross_entropy).  Kernel-level timings, the other
configurations (C2 contrastive 64x64, C3 padded rerank docs/s, C4 packed
pairs) and the CPU baseline are extra fields.

Before the W warmup steps, untimed C5 training steps run for --settle-ms
(default 500 ms), since the GPU clock ramps up over the first few hundred ms
of sustained load; the K timed steps are then full steps at the steady clock.

    python bench.py [--steps K] [--warmup W] [--settle-ms MS] [--quick] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E

# HBM-side bytes per launch of the forward kernel at C5, from the two
# rocprofv3 counter passes in profiles/c5_ops_hbm_traffic.md (FETCH_SIZE and
# WRITE_SIZE per dispatch, each scaled by what the counter reads for this
# build's own pack_rows_kernel copying 1 GiB: FETCH x1.997, WRITE x1.000).
# Counters cannot be read from inside this process, so the figure is the
# committed measurement, not a live one.
FWD_TRAFFIC_BYTES_C5 = int((52939.0 * 1.997 + 33888.4 * 1.000) * 1024)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-ms", type=float, default=500.0,
                   help="untimed C5 training steps for this long before the warmup steps: the "
                        "GPU clock ramps up over the first few hundred ms of sustained load")
    p.add_argument("--quick", action="store_true", help="headline workload only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--profile-ops", action="store_true",
                   help="run only the C5 operators (3x forward+argmax, 3x backward, 3x typed "
                        "backward) and two calibration kernels of known bytes, for rocprofv3 "
                        "counter passes")
    p.add_argument("--matrix", metavar="OUT_JSON",
                   help="run the reference's preset matrix (scripts/bench_matrix.py) instead and "
                        "write its v2 result schema to OUT_JSON")
    p.add_argument("--matrix-iters", type=int, default=30)
    p.add_argument("--matrix-repeats", type=int, default=3)
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# Workload generators (device-resident, seeded)
# ---------------------------------------------------------------------------
def make_c5(torch, dev, seed=0, nq=512, nb=512, lq=32, dim=128, lo=128, hi=1024, dup=0.01):
    F = torch.nn.functional
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (nb,), generator=g)
    total = int(lens.sum())
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    q = F.normalize(torch.randn(nq, lq, dim, generator=gd, device=dev), dim=-1)
    d = F.normalize(torch.randn(total, dim, generator=gd, device=dev), dim=-1)
    off = torch.zeros(nb + 1, dtype=torch.int64)
    off[1:] = lens.cumsum(0)
    if dup > 0:
        # overwrite 1% of document tokens with a copy of an earlier token of
        # the same document (exact ties; the lowest index must win)
        ndup = int(total * dup)
        doc = torch.randint(0, nb, (ndup,), generator=g)
        start, ln = off[doc], lens[doc]
        pos = (torch.rand(ndup, generator=g) * (ln - 1)).long() + 1
        src = (torch.rand(ndup, generator=g) * pos).long()
        d[(start + pos).to(dev)] = d[(start + src).to(dev)]
    return (q.to(torch.bfloat16), d.to(torch.bfloat16), off.to(torch.int32).to(dev),
            lens.tolist())


def make_c3(torch, dev, seed=0, B=256, C=1000, lq=32, ld=300, dim=128, only=None):
    """C3 inputs; ``only`` = list of query indices generates just those
    queries (bit-identical to the same rows of the full set)."""
    F = torch.nn.functional
    g = torch.Generator().manual_seed(seed)
    dlen = torch.randint(32, ld + 1, (B, C), generator=g, dtype=torch.int32)
    rows = list(range(B)) if only is None else list(only)
    q = torch.empty(len(rows), lq, dim, dtype=torch.float16, device=dev)
    d = torch.empty(len(rows), C, ld, dim, dtype=torch.float16, device=dev)
    for k, b in enumerate(rows):  # chunk-seeded so any query subset is reproducible
        gb = torch.Generator(device=dev).manual_seed(seed * 100003 + b)
        q[k] = F.normalize(torch.randn(lq, dim, generator=gb, device=dev), dim=-1).half()
        d[k] = F.normalize(torch.randn(C, ld, dim, generator=gb, device=dev), dim=-1).half()
    qlen = torch.full((len(rows),), lq, dtype=torch.int32, device=dev)
    return q, d, qlen, dlen[rows].to(dev)


def make_c4(torch, dev, seed=0, nq=512, nd=8192, npairs=20000, dim=128):
    F = torch.nn.functional
    g = torch.Generator().manual_seed(seed)
    ql = torch.randint(8, 65, (nq,), generator=g)
    dl = torch.exp(torch.randn(nd, generator=g) * 0.6 + torch.log(torch.tensor(180.0)))
    dl = dl.round().clamp(16, 2048).long()
    qoff = torch.zeros(nq + 1, dtype=torch.int32)
    qoff[1:] = ql.cumsum(0)
    doff = torch.zeros(nd + 1, dtype=torch.int32)
    doff[1:] = dl.cumsum(0)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    q = F.normalize(torch.randn(int(ql.sum()), dim, generator=gd, device=dev), dim=-1)
    d = F.normalize(torch.randn(int(dl.sum()), dim, generator=gd, device=dev), dim=-1)
    qids = torch.randint(0, nq, (npairs,), generator=g, dtype=torch.int32)
    dids = torch.randint(0, nd, (npairs,), generator=g, dtype=torch.int32)
    dscore = torch.randn(npairs, generator=g)
    return (q.bfloat16(), qoff.to(dev), d.bfloat16(), doff.to(dev), qids.to(dev),
            dids.to(dev), int(ql.max()), dscore.to(dev), ql, dl, qids, dids)


# ---------------------------------------------------------------------------
# Timing helpers
# ---------------------------------------------------------------------------
def time_events(torch, fn, reps, warmup):
    """Average ms per call with HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def time_wall(torch, fn, reps, warmup):
    """Average wall-clock ms per call of a host-synchronising API call,
    after ``warmup`` calls, with the device drained on both sides."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / reps


def cpu_model() -> str:
    """The host CPU as ``lscpu`` names it (model name, vendor, family/model/
    stepping, logical CPUs, hypervisor), else /proc/cpuinfo's model name."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        info = {}
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
        if info.get("Model name"):
            parts = [info["Model name"]]
            if info.get("Vendor ID"):
                parts.append(info["Vendor ID"])
            fms = "/".join(info.get(k, "?") for k in ("CPU family", "Model", "Stepping"))
            parts.append(f"family/model/stepping {fms}")
            if info.get("CPU(s)"):
                parts.append(f"{info['CPU(s)']} logical CPUs")
            if info.get("Hypervisor vendor"):
                parts.append(f"hypervisor {info['Hypervisor vendor']}")
            return ", ".join(parts)
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def make_c1(torch, dev, seed=0, nq=8, C=16, lq=32, ld=300, dim=128):
    """C1: padded rerank, fp32, Nq=8 x C=16, Lq=32, Ld padded to 300 with
    lengths U[64, 300], L2-normalised Gaussian rows."""
    F = torch.nn.functional
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(nq, lq, dim, generator=g), dim=-1)
    d = F.normalize(torch.randn(nq, C, ld, dim, generator=g), dim=-1)
    dlen = torch.randint(64, ld + 1, (nq, C), generator=g, dtype=torch.int32)
    qlen = torch.full((nq,), lq, dtype=torch.int32)
    return q.to(dev), d.to(dev), qlen.to(dev), dlen.to(dev)


def cpu_median(fn, reps, warmup):
    """Median wall seconds of ``reps`` calls after ``warmup`` calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def profile_ops(torch, dev):
    """The C5 operators in isolation (3x forward with argmax, 3x the fp32
    backward operator, 3x the typed backward of the training step), the C4
    packed forward (3x document-major, 3x pair kernel), then two
    of this build's own kernels whose HBM bytes are known exactly, to
    calibrate the FETCH_SIZE / WRITE_SIZE counters to bytes:

    * ``pack_rows_kernel`` copying 1 GiB of bf16 rows (every row valid):
      reads 1 GiB and writes 1 GiB, each byte once, 16-byte accesses;
    * ``pair_kernel`` (padded forward) over 1 GiB of fp16 candidate rows, all
      lengths full: reads the candidates once (plus 0.25 MiB of queries) and
      writes only the scores."""
    from maxsim_amd._ops import ops

    q, d, off, _ = make_c5(torch, dev)
    nq = q.shape[0]
    for _ in range(3):
        scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    dscore = (torch.softmax(scores, dim=1) - torch.eye(nq, device=dev)) / nq
    for _ in range(3):
        ops.maxsim_contrastive_backward(dscore, q, d, off, argmax)
    for _ in range(3):
        ops.maxsim_contrastive_backward_typed(dscore, q, d, off, argmax)
    del q, d, scores, argmax
    # C4 packed forward: 3x through the operator (document-major: grouping,
    # then doc_chunk_kernel), 3x through the C ABI entry point without a
    # workspace (pair_ring_kernel), the path C4 took before
    (q4, qo4, d4, do4, qi4, di4, mql, *_rest) = make_c4(torch, dev)
    for _ in range(3):
        ops.maxsim_packed_forward_with_argmax(q4, qo4, d4, do4, qi4, di4, mql)
    import ctypes
    from maxsim_amd._ops import NATIVE_LIB
    fn = ctypes.CDLL(str(NATIVE_LIB)).maxsim_amd_packed_forward_with_argmax
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    fn.argtypes = [ctypes.c_int, P, I64, P, I64, P, I64, P, I64, P, P, I64, I64, I64, P, P, P]
    s4 = torch.empty(qi4.numel(), device=dev)
    a4 = torch.empty(qi4.numel(), mql, dtype=torch.int32, device=dev)
    for _ in range(3):
        rc = fn(2, q4.data_ptr(), q4.shape[0], qo4.data_ptr(), qo4.numel() - 1, d4.data_ptr(),
                d4.shape[0], do4.data_ptr(), do4.numel() - 1, qi4.data_ptr(), di4.data_ptr(),
                qi4.numel(), q4.shape[1], mql, s4.data_ptr(), a4.data_ptr(),
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc
    del q4, d4, s4, a4
    # calibration 1: a 1 GiB row copy through pack_rows_kernel
    seg, ld, dim = 4096, 1024, 128
    padded = torch.randn(seg * ld, dim, device=dev).to(torch.bfloat16)
    lens = torch.full((seg,), ld, dtype=torch.int32, device=dev)
    offs = torch.arange(0, (seg + 1) * ld, ld, dtype=torch.int32, device=dev)
    for _ in range(3):
        ops.maxsim_pack_padded_rows(padded, lens, offs, ld, seg * ld)
    copy_bytes = padded.numel() * 2
    del padded
    # calibration 2: the padded forward reading 1 GiB of candidates once
    B, C, Lq, Ld = 64, 256, 32, 256
    qp = torch.randn(B * Lq, dim, device=dev).half()
    dp = torch.randn(B * C * Ld, dim, device=dev).half()
    ql = torch.full((B,), Lq, dtype=torch.int32, device=dev)
    dl = torch.full((B * C,), Ld, dtype=torch.int32, device=dev)
    for _ in range(3):
        ops.maxsim_padded_forward(qp, ql, dp, dl, Lq, Ld, C)
    torch.cuda.synchronize()
    print(json.dumps({"profile_ops": "c5", "pack_copy_bytes": copy_bytes,
                      "padded_read_bytes": dp.numel() * 2 + qp.numel() * 2,
                      "padded_write_bytes": B * C * 4}), flush=True)


# ---------------------------------------------------------------------------
# Preset matrix in the reference's bench_results/v2 schema
# (reference scripts/bench_matrix.py:291-545, 649-792): the same presets,
# timing (per-iteration events around one call, median over iterations, then
# the median over repeats), pure-PyTorch fp32 baselines, tolerances and
# fields, so a result file reads side by side with the reference's.
# ---------------------------------------------------------------------------
MATRIX_CONTRASTIVE = [("Contrastive", dict(Nq=32, Nb=32, Lq=32, Ld=80, dim=128)),
                      ("LongDocs", dict(Nq=32, Nb=32, Lq=32, Ld=512, dim=128)),
                      ("BigBatch", dict(Nq=64, Nb=64, Lq=32, Ld=128, dim=128))]
MATRIX_PADDED = [("Rerank", dict(B=32, C=50, Lq=32, Ld=180, dim=128)),
                 ("HeavyRerank", dict(B=32, C=100, Lq=32, Ld=256, dim=128))]
MATRIX_PACKED = [("PackedRerank", dict(B=32, C=50, Lq=32, Ld=180, dim=128)),
                 ("PackedHeavyRerank", dict(B=32, C=100, Lq=32, Ld=256, dim=128))]


def git_state() -> dict:
    """The commit this tree was built from: git where the metadata is
    present, else the record the native build wrote next to the libraries
    (maxsim_amd/_build_info.json), else unknown."""
    import subprocess

    try:
        head = subprocess.run(["git", "-C", str(ROOT), "rev-parse", "HEAD"], capture_output=True,
                              text=True, timeout=20)
        if head.returncode == 0:
            st = subprocess.run(["git", "-C", str(ROOT), "status", "--porcelain", "--",
                                 "maxsim_amd", "include", "oracle", "bench.py"],
                                capture_output=True, text=True, timeout=20)
            return {"git_commit": head.stdout.strip(),
                    "git_dirty": st.returncode == 0 and bool(st.stdout.strip())}
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        info = json.loads((ROOT / "maxsim_amd" / "_build_info.json").read_text())
        return {"git_commit": str(info.get("git_commit", "unknown")),
                "git_dirty": bool(info.get("git_dirty", False))}
    except (OSError, ValueError):
        return {"git_commit": "unknown", "git_dirty": False}


def matrix_payload(runs, *, machine, n_iter, n_warm, repeats, started, wall) -> dict:
    """The reference's v2 result record (scripts/bench_matrix.py:767-792)
    from ``runs`` (one list of per-preset measurements per repeat): medians
    over the repeats, backward time = step - forward, speedups and their
    spread across repeats."""
    def med(xs):
        xs = [x for x in xs if x is not None]
        return statistics.median(xs) if xs else None

    def ratio(a, b):
        return a / b if a is not None and b not in (None, 0) else None

    results = []
    for w in range(len(runs[0])):
        per = [r[w] for r in runs]
        base = per[0]
        k, n = med([r["k"] for r in per]), med([r["n"] for r in per])
        kf, nf = med([r["kf"] for r in per]), med([r["nf"] for r in per])
        kb = max(k - kf, 0.0) if kf is not None else None
        nb = max(n - nf, 0.0) if nf is not None else None
        kmb, nmb = med([r["kmb"] for r in per]), med([r["nmb"] for r in per])
        speedups = [r["n"] / r["k"] for r in per]
        variance = ({"step_speedup_min": min(speedups), "step_speedup_max": max(speedups),
                     "step_speedup_spread": max(speedups) - min(speedups),
                     "step_speedup_stdev": statistics.stdev(speedups), "n_repeats": len(per)}
                    if len(per) >= 2 else {"n_repeats": len(per)})
        results.append({
            "surface": base["surface"], "preset": base["preset"], "description": "",
            "shape": base["shape"], "dtype": base["dtype"],
            "maxsim_step_ms": k, "naive_step_ms": n, "step_speedup": ratio(n, k),
            "maxsim_fwd_ms": kf, "naive_fwd_ms": nf,
            "padded_ms": med([r["padded"] for r in per]),
            "maxsim_bwd_ms": kb, "naive_bwd_ms": nb, "bwd_speedup": ratio(nb, kb),
            "maxsim_peak_mb": kmb, "naive_peak_mb": nmb, "peak_ratio": ratio(nmb, kmb),
            "retained_reduction": base["red"], "correct": all(r["correct"] for r in per),
            "note": "", "variance": variance,
        })
    return {
        "schema_version": 1,
        "kernel": {"repo": "maxsim-mi355x", "version": 2, **git_state()},
        "machine": machine,
        "bench": {"iters_per_repeat": n_iter, "warmup": n_warm, "repeats": repeats,
                  "started_at": started, "wall_seconds": round(wall, 1)},
        "results": results,
    }


def run_matrix(args, torch, dev):
    import datetime
    import gc
    import maxsim_amd

    def time_step(fn, n_iter, n_warmup):
        for _ in range(n_warmup):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(n_iter):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        return statistics.median(times)

    def peak_mb(fn):
        gc.collect()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        fn()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() / 2**20

    def naive_contrastive(q, docs, cu, d_lens):
        nb, ld = len(d_lens), max(d_lens)
        padded = docs.new_zeros((nb, ld, q.shape[2]))
        offs = cu.to(torch.int64).cpu().tolist()
        for i, n in enumerate(d_lens):
            padded[i, :n] = docs[offs[i]:offs[i + 1]]
        sim = torch.einsum("qid,njd->qnij", q.float(), padded.float())
        return sim.max(dim=-1).values.sum(dim=-1)

    def naive_padded(q, d, qlen, dlen):
        lq, ld = q.shape[1], d.shape[2]
        sim = torch.einsum("bid,bcjd->bcij", q.float(), d.float())
        qm = torch.arange(lq, device=q.device)[None, :] < qlen[:, None]
        dm = torch.arange(ld, device=q.device)[None, None, :] < dlen[:, :, None]
        best = sim.masked_fill(~dm[:, :, None, :], float("-inf")).max(dim=-1).values
        return best.masked_fill(~qm[:, None, :], 0.0).sum(dim=-1)

    def close(a, b):
        return bool(torch.allclose(a.float(), b.float(), rtol=3e-2, atol=3e-2))

    label = {torch.float16: "fp16", torch.bfloat16: "bf16"}
    n_iter, n_warm = args.matrix_iters, 5

    def contrastive(name, shape, dtype):
        g = torch.Generator().manual_seed(1234)
        Nq, Nb, Lq, Ld, D = shape["Nq"], shape["Nb"], shape["Lq"], shape["Ld"], shape["dim"]
        q = torch.randn(Nq, Lq, D, generator=g, dtype=dtype).to(dev)
        docs = torch.randn(Nb * Ld, D, generator=g, dtype=dtype).to(dev)
        cu = torch.arange(0, (Nb + 1) * Ld, Ld, dtype=torch.int32, device=dev)
        lens = [Ld] * Nb

        def fresh():
            return (q.detach().clone().requires_grad_(True),
                    docs.detach().clone().requires_grad_(True))

        def k_step():
            a, b = fresh()
            maxsim_amd.score_contrastive_train(a, b, cu).sum().backward()

        def n_step():
            a, b = fresh()
            naive_contrastive(a, b, cu, lens).sum().backward()

        def k_fwd():
            a, b = fresh()
            return maxsim_amd.score_contrastive_train(a, b, cu)

        def n_fwd():
            a, b = fresh()
            return naive_contrastive(a, b, cu, lens)

        qk, dk = fresh()
        qn, dn = fresh()
        maxsim_amd.score_contrastive_train(qk, dk, cu).sum().backward()
        naive_contrastive(qn, dn, cu, lens).sum().backward()
        ok = close(qk.grad, qn.grad) and close(dk.grad, dn.grad)
        return dict(surface="contrastive_train", preset=name,
                    shape={"Nq": Nq, "Nb": Nb, "Lq": Lq, "Ld": Ld, "D": D}, dtype=label[dtype],
                    k=time_step(k_step, n_iter, n_warm), n=time_step(n_step, n_iter, n_warm),
                    kf=time_step(k_fwd, n_iter, n_warm), nf=time_step(n_fwd, n_iter, n_warm),
                    padded=None, kmb=peak_mb(k_step), nmb=peak_mb(n_step), red=float(Ld),
                    correct=ok)

    def padded_inputs(shape, dtype):
        g = torch.Generator().manual_seed(1234)
        B, C, Lq, Ld, D = shape["B"], shape["C"], shape["Lq"], shape["Ld"], shape["dim"]
        q = torch.randn(B, Lq, D, generator=g, dtype=dtype).to(dev)
        d = torch.randn(B, C, Ld, D, generator=g, dtype=dtype).to(dev)
        qlen = torch.full((B,), Lq, dtype=torch.int32, device=dev)
        dlen = torch.full((B, C), Ld, dtype=torch.int32, device=dev)
        return q, d, qlen, dlen, {"B": B, "K": C, "Lq": Lq, "Ld": Ld, "D": D}

    def padded(name, shape, dtype):
        q, d, qlen, dlen, sh = padded_inputs(shape, dtype)

        def k_step():
            return maxsim_amd.score_candidates_padded(q, d, qlen, dlen)

        def n_step():
            return naive_padded(q, d, qlen, dlen)

        ok = close(k_step(), n_step())
        return dict(surface="padded_infer", preset=name, shape=sh, dtype=label[dtype],
                    k=time_step(k_step, n_iter, n_warm), n=time_step(n_step, n_iter, n_warm),
                    kf=None, nf=None, padded=None, kmb=peak_mb(k_step), nmb=peak_mb(n_step),
                    red=None, correct=ok)

    def packed(name, shape, dtype):
        q, d, qlen, dlen, sh = padded_inputs(shape, dtype)
        B, C, Lq, Ld, D = sh["B"], sh["K"], sh["Lq"], sh["Ld"], sh["D"]
        qf, df = q.reshape(B * Lq, D).contiguous(), d.reshape(B * C * Ld, D).contiguous()
        qoff = torch.arange(0, (B + 1) * Lq, Lq, dtype=torch.int32, device=dev)
        doff = torch.arange(0, (B * C + 1) * Ld, Ld, dtype=torch.int32, device=dev)
        dids = torch.arange(B * C, dtype=torch.int32, device=dev)
        qids = dids // C

        def k_step():
            return maxsim_amd.score_pairs_packed(qf, qoff, df, doff, qids, dids, max_q_len=Lq)

        def n_step():
            return naive_padded(q, d, qlen, dlen)

        def p_step():
            return maxsim_amd.score_candidates_padded(q, d, qlen, dlen)

        sk = k_step().view(B, C)
        ok = close(sk, p_step()) and close(sk, n_step())
        return dict(surface="packed_infer", preset=name, shape=sh, dtype=label[dtype],
                    k=time_step(k_step, n_iter, n_warm), n=time_step(n_step, n_iter, n_warm),
                    kf=None, nf=None, padded=time_step(p_step, n_iter, n_warm),
                    kmb=peak_mb(k_step), nmb=peak_mb(n_step), red=None, correct=ok)

    def one_matrix():
        rs = []
        for dtype in (torch.float16, torch.bfloat16):
            rs += [contrastive(n, s, dtype) for n, s in MATRIX_CONTRASTIVE]
            rs += [padded(n, s, dtype) for n, s in MATRIX_PADDED]
            rs += [packed(n, s, dtype) for n, s in MATRIX_PACKED]
            log(f"matrix: {label[dtype]} done")
        return rs

    started = datetime.datetime.now(datetime.timezone.utc)
    t0 = time.perf_counter()
    runs = [one_matrix() for _ in range(args.matrix_repeats)]
    wall = time.perf_counter() - t0
    props = torch.cuda.get_device_properties(dev)
    machine = {"gpu_name": torch.cuda.get_device_name(dev),
               "compute_capability": getattr(props, "gcnArchName", "gfx950"),
               "torch_version": torch.__version__,
               "cuda_version": getattr(torch.version, "hip", None)}
    payload = matrix_payload(runs, machine=machine, n_iter=n_iter, n_warm=n_warm,
                             repeats=args.matrix_repeats,
                             started=started.strftime("%Y-%m-%dT%H:%M:%SZ"), wall=wall)
    results = payload["results"]
    with open(args.matrix, "w") as f:
        f.write(json.dumps(payload, indent=2) + "\n")
    log(f"matrix: wrote {args.matrix}")
    for r in results:
        log(f"{r['surface']:18s} {r['preset']:18s} {r['dtype']}  maxsim {r['maxsim_step_ms']:.4f} ms  "
            f"naive {r['naive_step_ms']:.4f} ms  correct {r['correct']}")
    return 0 if all(r["correct"] for r in results) else 1


def main():
    args = parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the contrastive batch would shard by query rows); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import torch.nn.functional as F

    import maxsim_amd
    from maxsim_amd._ops import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.matrix:
        sys.exit(run_matrix(args, torch, dev))
    if args.profile_ops:
        profile_ops(torch, dev)
        return
    K, W = args.steps, args.warmup
    extra = {}

    # ---------------- C5: headline contrastive training step ----------------
    log("C5: generating inputs")
    q, d, off, lens = make_c5(torch, dev)
    nq, lq, dim = q.shape
    nb = off.numel() - 1
    total = d.shape[0]
    flops_fwd = 2.0 * dim * nq * lq * total
    target = torch.arange(nq, device=dev)

    qg = q.clone().requires_grad_(True)
    dg = d.clone().requires_grad_(True)

    def step():
        qg.grad = None
        dg.grad = None
        scores = maxsim_amd.score_contrastive_train(qg, dg, off)
        loss = F.cross_entropy(scores, target)
        loss.backward()
        return loss

    # Settle: the clock ramps up over the first few hundred ms of sustained
    # load (one box: the C5 forward at 1.05 ms 30 ms into a run, 0.99 ms at
    # 360 ms), so untimed training steps run for settle_ms before the W
    # warmup steps, and the K timed steps see the steady clock.
    n_settle = 0
    t_settle = time.perf_counter() + args.settle_ms / 1e3
    while time.perf_counter() < t_settle:
        step()
        n_settle += 1
    torch.cuda.synchronize()
    log(f"C5: settle {n_settle} steps ({args.settle_ms:.0f} ms), warmup {W} steps (T_d={total})")
    for _ in range(W):
        step()
    torch.cuda.synchronize()
    log(f"C5: timing {K} steps")
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / K

    # the same step through the fused loss (softmax gradient recomputed inside
    # the backward kernels, no dscore tensor, no autograd graph for the loss)
    def step_fused():
        qg.grad = None
        dg.grad = None
        loss = maxsim_amd.score_contrastive_cross_entropy(qg, dg, off)
        loss.backward()
        return loss

    for _ in range(W):
        step_fused()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(K):
        step_fused()
    torch.cuda.synchronize()
    ms_step_fused = (time.perf_counter() - t0) * 1e3 / K

    # kernel-level (op calls, no Python validation)
    ms_fwd = time_events(torch, lambda: ops.maxsim_contrastive_forward_with_argmax(q, d, off), K, 2)
    scores, argmax = ops.maxsim_contrastive_forward_with_argmax(q, d, off)
    dscore = (torch.softmax(scores, dim=1) - torch.eye(nq, device=dev)) / nq
    # 30 untimed calls first (~8 ms): right after the forward timing the clock
    # is still at the MFMA phase's level, and the backward runs ~10 % slower
    # for the first ~20 ms (one box: 282, 269, 261, 253 us in successive
    # 20-call windows with 2 warmups each).
    ms_bwd = time_events(torch, lambda: ops.maxsim_contrastive_backward(dscore, q, d, off, argmax), K, 30)
    ms_fwd_scoreonly = time_events(torch, lambda: ops.maxsim_contrastive_forward(q, d, off), K, 2)
    bytes_bwd = (4 * nq * nb * lq + 4 * nq * nb + 2 * dim * (nq * lq + total)
                 + 4 * dim * (nq * lq + total))
    fwd_tflops = flops_fwd / (ms_fwd * 1e-3) / 1e12
    extra["c5"] = {
        "T_d": total, "flops_fwd": flops_fwd,
        "settle_ms": args.settle_ms, "settle_steps": n_settle,
        "step_ms": round(ms_step, 4),
        "fused_ce_step_ms": round(ms_step_fused, 4),
        "fwd_ms": round(ms_fwd, 4), "fwd_tflops": round(fwd_tflops, 2),
        "fwd_scoreonly_ms": round(ms_fwd_scoreonly, 4),
        "bwd_ms": round(ms_bwd, 4), "bwd_bytes": bytes_bwd,
        "bwd_gbps": round(bytes_bwd / (ms_bwd * 1e-3) / 1e9, 1),
        "bwd_hbm_frac": round(bytes_bwd / (ms_bwd * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        "kernel_step_ms": round(ms_fwd + ms_bwd, 4),
    }
    log(f"C5: step {ms_step:.3f} ms, fwd {ms_fwd:.3f} ms ({fwd_tflops:.1f} TFLOP/s), bwd {ms_bwd:.3f} ms")

    # One GPU's shard of C5 split by query rows over 8 GPUs (64 of the 512
    # queries against all 512 documents): the kernels at the shape each rank
    # would run, without the collectives (one GPU here).
    # (not in --quick, whose kernel trace averages the full-size C5 forward)
    if not args.quick:
        qs = q[:64].contiguous()
        ms_sf = time_events(torch, lambda: ops.maxsim_contrastive_forward_with_argmax(qs, d, off),
                            K, 2)
        s_s, a_s = ops.maxsim_contrastive_forward_with_argmax(qs, d, off)
        g_s = dscore[:64].contiguous()
        ms_sb = time_events(torch, lambda: ops.maxsim_contrastive_backward_typed(
            g_s, qs, d, off, a_s), K, 2)
        extra["c5_shard_of_8"] = {"Nq": 64, "Nb": nb, "fwd_ms": round(ms_sf, 4),
                                  "fwd_tflops": round(flops_fwd / 8 / (ms_sf * 1e-3) / 1e12, 2),
                                  "bwd_typed_ms": round(ms_sb, 4)}
        del s_s, a_s

    if not args.quick:
        # ---------------- C1: small padded rerank, fp32 ----------------
        log("C1: padded rerank 8x16, fp32")
        q1, d1, ql1, dl1 = make_c1(torch, dev)
        B1, C1_, Lq1, Ld1 = d1.shape[0], d1.shape[1], q1.shape[1], d1.shape[2]
        qf1, df1 = q1.reshape(B1 * Lq1, -1), d1.reshape(B1 * C1_ * Ld1, -1)
        dlf1 = dl1.reshape(-1)
        ms1k = time_events(torch, lambda: ops.maxsim_padded_forward_with_argmax(
            qf1, ql1, df1, dlf1, Lq1, Ld1, C1_), K, 2)
        ms1a = time_wall(torch, lambda: maxsim_amd.score_candidates_padded_with_argmax(
            q1, d1, ql1, dl1), K, 2)
        extra["c1"] = {"kernel_ms": round(ms1k, 4), "api_call_ms": round(ms1a, 4)}

        # ---------------- C2: small contrastive step ----------------
        log("C2: contrastive 64x64")
        q2, d2, off2, lens2 = make_c5(torch, dev, seed=1, nq=64, nb=64, lo=64, hi=512, dup=0.0)
        q2g, d2g = q2.clone().requires_grad_(True), d2.clone().requires_grad_(True)
        t2 = torch.arange(64, device=dev)

        def step2():
            q2g.grad = None
            d2g.grad = None
            F.cross_entropy(maxsim_amd.score_contrastive_train(q2g, d2g, off2), t2).backward()

        ms2 = time_wall(torch, step2, K, W)

        # loss and gradients in one call, without the autograd engine
        def step2_vg():
            maxsim_amd.score_contrastive_cross_entropy_value_and_grad(q2, d2, off2)

        ms2_vg = time_wall(torch, step2_vg, K, W)

        def step2_fused():
            q2g.grad = None
            d2g.grad = None
            maxsim_amd.score_contrastive_cross_entropy(q2g, d2g, off2).backward()

        # host checks off: no call waits for the device (the kernels flag
        # invalid layouts with NaN scores instead)
        with maxsim_amd.host_checks(False):
            ms2_nowait = time_wall(torch, step2, K, W)
            ms2_fused_nowait = time_wall(torch, step2_fused, K, W)
            ms2_vg_nowait = time_wall(torch, step2_vg, K, W)
            # the same step captured once in a HIP graph and replayed
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step2()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            q2g.grad = None
            d2g.grad = None
            with torch.cuda.graph(graph):
                F.cross_entropy(maxsim_amd.score_contrastive_train(q2g, d2g, off2), t2).backward()
            ms2_graph = time_wall(torch, graph.replay, K, W)
            del graph
        q2g.grad = None
        d2g.grad = None
        extra["c2"] = {"step_ms": round(ms2, 4),
                       "no_host_checks_step_ms": round(ms2_nowait, 4),
                       "fused_ce_no_host_checks_step_ms": round(ms2_fused_nowait, 4),
                       "value_and_grad_step_ms": round(ms2_vg, 4),
                       "value_and_grad_no_host_checks_step_ms": round(ms2_vg_nowait, 4),
                       "graph_step_ms": round(ms2_graph, 4),
                       "fwd_ms": round(time_events(torch, lambda: ops.maxsim_contrastive_forward_with_argmax(q2, d2, off2), K, 2), 4)}
        log(f"C2: step {ms2:.4f} ms; host checks off {ms2_nowait:.4f} ms, fused "
            f"{ms2_fused_nowait:.4f} ms, graph {ms2_graph:.4f} ms, value_and_grad "
            f"{ms2_vg:.4f} ms ({ms2_vg_nowait:.4f} ms host checks off)")

        # ---------------- C3: padded rerank docs/s ----------------
        log("C3: padded rerank 256x1000 (19.7 GB fp16)")
        q3, d3, ql3, dl3 = make_c3(torch, dev)
        B, C, Ld = d3.shape[0], d3.shape[1], d3.shape[2]
        qf = q3.reshape(B * 32, 128)
        df = d3.reshape(B * C * Ld, 128)
        dlf = dl3.reshape(-1)
        ms3 = time_events(torch, lambda: ops.maxsim_padded_forward(qf, ql3, df, dlf, 32, Ld, C), max(3, K // 4), 1)
        real_rows = int(dl3.sum())
        bytes3 = 2 * 128 * (real_rows + B * 32) + 8 * B * C
        api3 = time_wall(torch, lambda: maxsim_amd.score_candidates_padded(q3, d3, ql3, dl3), 3, 1)
        extra["c3"] = {"kernel_ms": round(ms3, 4), "docs_per_s": round(B * C / (ms3 * 1e-3), 1),
                       "gbps": round(bytes3 / (ms3 * 1e-3) / 1e9, 1),
                       "hbm_frac": round(bytes3 / (ms3 * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                       "api_ms": round(api3, 3)}
        log(f"C3: {ms3:.3f} ms -> {B * C / (ms3 * 1e-3):.3e} docs/s")
        # padded -> packed copy of the same candidates (the device work of
        # _pack_padded): 2 x the valid rows' bytes
        doff3 = torch.zeros(B * C + 1, dtype=torch.int32, device=dev)
        doff3[1:] = dlf.cumsum(0)
        ms_pack = time_events(torch, lambda: ops.maxsim_pack_padded_rows(df, dlf, doff3, Ld, real_rows),
                              max(3, K // 4), 1)
        bytes_pack = 2 * 2 * 128 * real_rows
        extra["c3_pack"] = {"kernel_ms": round(ms_pack, 4),
                            "gbps": round(bytes_pack / (ms_pack * 1e-3) / 1e9, 1),
                            "hbm_frac": round(bytes_pack / (ms_pack * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"C3 pack: {ms_pack:.3f} ms, {bytes_pack / (ms_pack * 1e-3) / 1e9:.0f} GB/s")
        # padded training backward over the first 16 candidates of each C3
        # query (not a BASELINE configuration): gradients written in fp16 by
        # the autograd path's operator, against the fp32 operator plus the
        # cast that autograd applies after the reference's backward
        Ct = 16
        dtf = d3[:, :Ct].contiguous().reshape(B * Ct * Ld, 128)
        dltf = dl3[:, :Ct].contiguous().reshape(-1)
        _, amt = ops.maxsim_padded_forward_with_argmax(qf, ql3, dtf, dltf, 32, Ld, Ct)
        gt = torch.randn(B * Ct, generator=torch.Generator(device=dev).manual_seed(3), device=dev)
        bargs = (gt, qf, dtf, ql3, dltf, amt, 32, Ld, Ct)

        def cast_route():
            dq_, dd_ = ops.maxsim_padded_backward(*bargs)
            return dq_.half(), dd_.half()

        ms_bt = time_events(torch, lambda: ops.maxsim_padded_backward_typed(*bargs), K, 2)
        ms_bc = time_events(torch, cast_route, K, 2)
        # fp16 dQ and dD (padding rows included) written; Q read once, one
        # document row gathered per (candidate, token); argmax, dscore, lengths
        bytes_bt = (2 * 128 * (B * 32 + B * Ct * Ld) + 2 * 128 * (B * 32 + B * Ct * 32)
                    + 4 * (B * Ct * 32 + 2 * B * Ct + B))
        extra["c3_train_bwd"] = {"candidates": f"{B}x{Ct}", "typed_ms": round(ms_bt, 4),
                                 "fp32_plus_cast_ms": round(ms_bc, 4),
                                 "typed_gbps": round(bytes_bt / (ms_bt * 1e-3) / 1e9, 1),
                                 "typed_hbm_frac": round(bytes_bt / (ms_bt * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"C3 train bwd ({B}x{Ct}): typed {ms_bt:.3f} ms, fp32 + cast {ms_bc:.3f} ms")
        del q3, d3, qf, df, dtf, amt
        torch.cuda.empty_cache()

        # ---------------- C4: packed pairs fwd + bwd ----------------
        log("C4: packed 20k pairs")
        (q4, qo4, d4, do4, qi4, di4, mql, g4, *_rest) = make_c4(torch, dev)
        ms4f = time_events(torch, lambda: ops.maxsim_packed_forward_with_argmax(q4, qo4, d4, do4, qi4, di4, mql), K, 2)
        _, am4 = ops.maxsim_packed_forward_with_argmax(q4, qo4, d4, do4, qi4, di4, mql)
        ms4b = time_events(torch, lambda: ops.maxsim_packed_backward(g4, q4, qo4, d4, do4, qi4, di4, am4, mql), K, 2)
        q4g, d4g = q4.clone().requires_grad_(True), d4.clone().requires_grad_(True)

        def step4():
            q4g.grad = None
            d4g.grad = None
            s4 = maxsim_amd.score_pairs_packed_train(q4g, qo4, d4g, do4, qi4, di4, max_q_len=mql)
            s4.backward(g4)

        api4 = time_wall(torch, step4, K, 2)
        extra["c4"] = {"fwd_ms": round(ms4f, 4), "bwd_ms": round(ms4b, 4),
                       "api_train_step_ms": round(api4, 4)}

    # ---------------- CPU baseline ----------------
    # The reference's naive PyTorch formulation (einsum + max, fp32; autograd
    # for the backward) on the host's cores: C5 on a bounded sample of query
    # rows (the headline's cpu_baseline), C1 and C2 in full, C3 on a fixed
    # subset of queries, C4 on a fixed subset of pairs.
    cpu = None
    if not args.no_cpu:
        from oracle import torch_baseline

        # the GPU box's CPU share is 16 threads whatever the affinity mask shows
        cores = min(16, len(os.sched_getaffinity(0)))
        torch.set_num_threads(cores)
        host = cpu_model()
        nsample = 64
        qc = q[:nsample].float().cpu()
        dc, mask = torch_baseline.pad_documents(d.float().cpu(), lens)
        rows = torch.arange(nsample)
        log(f"CPU baseline: {nsample} of {nq} query rows x {nb} docs on {cores} threads ({host})")
        t_sample = cpu_median(lambda: torch_baseline.contrastive_step(qc, rows, dc, mask, nq), 5, 2)
        cpu_tflops = (flops_fwd * nsample / nq) / t_sample / 1e12
        cpu = {"value": round(cpu_tflops, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
               "sample": f"C5 fwd+CE+bwd for {nsample}/{nq} query rows against all {nb} docs "
                         f"(fp32 einsum+max, -inf masked padding to Ld_max), median of 5 after 2 warmups; "
                         f"{t_sample:.3f} s per sample step; host CPU: {host}",
               "step_ms_extrapolated": round(t_sample * nq / nsample * 1e3, 1),
               "host": host}
        log(f"CPU baseline: {t_sample:.3f} s per sample -> {cpu_tflops:.4f} TFLOP/s")
        if not args.quick:
            legs = {}
            # C1 in full: padded scores + argmax, fp32
            c1c = [t.cpu() for t in (q1, d1, ql1, dl1)]
            t1 = cpu_median(lambda: torch_baseline.padded_scores_with_argmax(*c1c), 5, 2)
            legs["c1"] = {"ms": round(t1 * 1e3, 3), "what": "padded fwd + argmax, 8x16, in full"}
            # C2 in full: fwd + CE(diagonal) + bwd
            dc2, mask2 = torch_baseline.pad_documents(d2.float().cpu(), lens2)
            q2c = q2.float().cpu()
            t2 = cpu_median(lambda: torch_baseline.contrastive_step(q2c, torch.arange(64), dc2,
                                                                    mask2, 64), 5, 2)
            legs["c2"] = {"step_ms": round(t2 * 1e3, 2), "what": "fwd+CE+bwd, 64x64, in full"}
            # C3 on queries 0, 97, 255 (chunk-seeded: bit-identical to those rows of the full set)
            sub = [0, 97, 255]
            q3s, d3s, ql3s, dl3s = make_c3(torch, dev, only=sub)
            c3c = (q3s.float().cpu(), d3s.float().cpu(), ql3s.cpu(), dl3s.cpu())
            del q3s, d3s
            t3 = cpu_median(lambda: torch_baseline.padded_scores(*c3c), 3, 1)
            legs["c3"] = {"docs_per_s": round(len(sub) * c3c[1].shape[1] / t3, 1),
                          "what": f"padded fwd, queries {sub} x 1000 candidates (fp16 inputs in fp32)"}
            # C4 on its first 2,000 pairs (the pair ids are uniform random):
            # fwd + bwd with the upstream gradient; the full step is ~10x
            n4 = 2000
            c4c = [t.cpu() for t in (q4, qo4, d4, do4, qi4[:n4], di4[:n4])]
            c4c[0], c4c[2] = c4c[0].float(), c4c[2].float()
            g4c = g4[:n4].cpu()
            t4 = cpu_median(lambda: torch_baseline.packed_step(*c4c, g4c), 3, 1)
            legs["c4"] = {"sample_step_ms": round(t4 * 1e3, 1),
                          "step_ms_extrapolated": round(t4 * 1e3 * qi4.numel() / n4, 1),
                          "what": f"packed fwd+bwd on the first {n4} of {qi4.numel()} pairs "
                                  "(pairs by document length, padded chunks)"}
            cpu["legs"] = legs
            log("CPU legs: " + ", ".join(f"{k} {v}" for k, v in legs.items()))

    value = flops_fwd / (ms_step * 1e-3) / 1e12
    out = {
        "metric": "contrastive fwd+bwd ms & MFMA TFLOP/s; rerank docs/sec at Lq=32 Ld=300 d=128",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded L2-normalised Gaussian embeddings, 1% duplicated doc tokens)",
        "config": {"workload": "C5 contrastive training step: Nq=Nb=512, Lq=32, Ld~U[128,1024], "
                               "dim=128, fwd + CE(diagonal) + bwd",
                   "Nq": nq, "Nb": nb, "Lq": lq, "dim": dim, "total_doc_tokens": total},
        "roofline": {"bound": "mfma", "kernel": "contrastive_tiled_kernel (forward + argmax)",
                     "achieved": round(fwd_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(fwd_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": FWD_TRAFFIC_BYTES_C5,
                     # algorithmic bytes of one forward launch: Q and D read,
                     # scores and argmax written, each once
                     "traffic_over_algorithmic": round(
                         FWD_TRAFFIC_BYTES_C5 / (2 * dim * (nq * lq + total) + 4 * nq * nb
                                                 + 4 * nq * nb * lq), 3),
                     "traffic_source": "profiles/c5_ops_hbm_traffic.md"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
