#!/usr/bin/env python3
"""Throughput of the fused NAR rotate -> rank-k -> INT4 path on one MI355X.

One step = one call of the fused operator over one batch of synthetic tokens
(default: the Llama-3.1-8B down_proj shape, 8192 x 14336 bf16, H_28 (x) H_512,
k=32, b=128).  Inputs are resident in HBM before the timed region; R input and
output buffers are rotated so that consecutive steps never reuse a buffer the
256 MB Infinity Cache could still hold.

Prints ONE JSON line (rank 0): tokens/s, achieved HBM GB/s from the algorithmic
byte model T*(2n + n/2 + 4n/b) + factor bytes, the roofline of the dominant
kernel (HIP-event timed on the stream it runs on) and the CPU baseline (the
reference's PyTorch op sequence on a bounded sample of the same rows).
"""

from __future__ import annotations

import argparse
import json
import ctypes
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "nar-offline-validation_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fused NAR+INT4 quant: tokens/s and achieved HBM GB/s (% peak), 1 MI355X"
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 << 20

# HBM bytes per call and MFMA busy fractions are measured with rocprofv3 counter
# runs of this script (the commands are in the profiles) and filed under the
# SHA-256 of the kernel sources they were taken on; a profile of other sources
# is reported as stale (null), never as a number for the current kernels.
TRAFFIC_SOURCE = ROOT / "profiles" / "hbm_traffic.md"
MFMA_UTIL_SOURCE = ROOT / "profiles" / "mfma_utilisation.md"


def _profile_sections(path: Path) -> dict[str, str]:
    """'## <config> ...' sections of a profile, keyed by config name."""
    if not path.exists():
        return {}
    out, cur = {}, None
    for line in path.read_text().splitlines():
        if line.startswith("## "):
            cur = line[3:].split()[0]
            out[cur] = ""
        elif cur:
            out[cur] += line + "\n"
    return out


def _sources_key(text: str) -> str | None:
    m = re.search(r"Kernel sources sha256: ([0-9a-f]{64})", text)
    return m.group(1) if m else None


def measured_traffic(config: str, sha: str) -> tuple[float | None, str]:
    """(HBM bytes per call, status) from the traffic profile of this config."""
    sec = _profile_sections(TRAFFIC_SOURCE).get(config)
    if sec is None:
        return None, "not profiled"
    if _sources_key(sec) != sha:
        return None, "stale: profiled on other kernel sources"
    m = re.search(r"Total per call: \*\*([0-9.]+) MB\*\*", sec)
    return (float(m.group(1)) * 1e6, "measured") if m else (None, "no total")


def measured_mfma_busy(config: str, sha: str) -> dict | None:
    """MFMA busy fraction per kernel of this config, or None if not profiled on these sources."""
    if not MFMA_UTIL_SOURCE.exists():
        return None
    text = MFMA_UTIL_SOURCE.read_text()
    if _sources_key(text) != sha:
        return None
    busy = {}
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == config and cells[3].endswith("%"):
            kernel = re.sub(r"[`<].*", "", cells[1].replace("void ", "").strip("` ")) or cells[1]
            busy[kernel] = float(cells[3].rstrip("%")) / 100.0
    return busy or None


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="downproj_8b",
                    choices=["kcache_3b", "qproj_3b", "downproj_8b", "vcache_decode_8b", "downproj_70b",
                             "e17_8b_k8", "e17_8b_k32", "e17_3b_k8", "e17_3b_k32", "e28_8b", "e28_3b",
                             "w4a4_8b", "hook_kcache_3b", "hook_rows_8192", "hook_rows_qwen3_8b"])
    ap.add_argument("--tokens", type=int, default=0,
                    help="token count of the e28_* transform settings (default 2048) and of w4a4_8b "
                         "(default 8192)")
    ap.add_argument("--rank-mode", default="auto", choices=["auto", "exact", "mfma"])
    ap.add_argument("--api", default="cabi", choices=["cabi", "op"],
                    help="time the C-ABI entry point (default) or the torch.ops.narhip operator")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU baseline work")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="instead of the workload, time a plain device copy of this many MiB (the "
                         "reference reading for the FETCH_SIZE / WRITE_SIZE byte counters)")
    return ap.parse_args()


def copy_calibration(mib: int, steps: int) -> int:
    import torch
    dev = torch.device("cuda:0")
    nbytes = mib << 20
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize(dev)
    ms = ev0.elapsed_time(ev1) / steps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "ms_per_copy": ms,
                      "gbps": 2 * nbytes / (ms * 1e-3) / 1e9}), flush=True)
    return 0


def describe(w) -> str:
    m, q = w.hadamard
    had = f"H{q} per block" if m == 1 else f"H{m}xH{q}"
    rb = "" if w.rank_block in (None, w.n) else f" per {w.rank_block}-block"
    return f"{w.name}: {w.tokens} tokens x {w.n} bf16, {had}, k={w.k}{rb}, b={w.group}"


def cpu_baseline(w, target_s: float) -> dict:
    import torch

    from oracle import torch_path
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rows = min(w.tokens, 16)

    def once(r: int) -> float:
        t0 = time.perf_counter()
        for lo in range(0, r, 1024):
            hi = min(r, lo + 1024)
            torch_path.run(w.x[lo:hi], *w.hadamard, w.v, w.w_t, w.group, w.rank_block)
        return time.perf_counter() - t0

    once(rows)
    dt = once(rows)
    while dt * 6 < target_s and rows < w.tokens:
        rows = min(w.tokens, rows * 2)
        dt = once(rows)
    times = [once(rows) for _ in range(5)]
    med = statistics.median(times)
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": rows / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {rows} of {w.tokens} rows of the same workload, torch CPU op sequence of the "
                      f"reference (oracle/torch_path.py), median of 5 after 1 warmup; cpu: {model}"}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: the path is row-independent and shards by tokens "
              "with no communication beyond a broadcast of the factors; run with --gpus 1.",
              file=sys.stderr)
        return 2

    if args.copy_mb:
        return copy_calibration(args.copy_mb, args.steps)

    import numpy as np
    import torch

    from narhip import _lib, ops, workloads
    from narhip.build import sources_sha256

    mode = {"auto": ops.RANK_AUTO, "exact": ops.RANK_EXACT, "mfma": ops.RANK_MFMA}[args.rank_mode]
    if args.config.startswith("hook_"):
        return bench_hook(args, torch.device("cuda:0"))
    if args.config == "w4a4_8b":
        return bench_w4a4(args, torch.device("cuda:0"))
    if args.config.startswith("e28_"):
        w = workloads.REFERENCE_SETTINGS[args.config](args.tokens or 2048)
    else:
        w = (workloads.CONFIGS.get(args.config) or workloads.REFERENCE_SETTINGS[args.config])()
    dev = torch.device("cuda:0")
    if w.transform_f16:
        return bench_transform_f16(args, w, dev)
    x_host = torch.from_numpy(w.x.view(np.int16))
    in_bytes = w.x.nbytes
    R = max(2, min(8, -(-2 * MALL_BYTES // max(in_bytes, 1)) + 1))
    xs = [x_host.to(dev).view(torch.bfloat16) for _ in range(R)]
    v = None if w.v is None else torch.from_numpy(w.v).to(dev)
    wt = None if w.w_t is None else torch.from_numpy(w.w_t).to(dev)
    rows_out = w.out_rows or w.tokens
    outs = [(torch.empty((rows_out, w.n // 2), dtype=torch.uint8, device=dev),
             torch.empty((rows_out, w.n // w.group), dtype=torch.float16, device=dev),
             torch.empty((rows_out, w.n // w.group), dtype=torch.float16, device=dev)) for _ in range(R)]
    dest = None if w.dest_rows is None else torch.from_numpy(w.dest_rows).to(dev)
    full_row_rank = w.k > 0 and w.rank_block in (None, w.n)
    # factor terms are prepared once per factor set, as the reference's modules do
    prepared = ops.prepare_rank_factors(v, wt, w.n, w.k) if full_row_rank and mode != ops.RANK_EXACT else None

    # The timed step calls the C ABI (include/narhip.h) directly: the drop-in
    # boundary of the path.  The torch.ops.narhip operator over the same entry
    # point adds 25-35 us of Python dispatch per call (--api op times that).
    lib = _lib.load()
    m, q = w.hadamard
    nb = w.n if w.rank_block is None else w.rank_block
    ws_bytes = lib.narhip_rotate_quant_workspace(w.tokens, w.n, m, q, w.k, nb, 0, 0, int(prepared is not None),
                                                 mode)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    cstream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def step(i: int) -> None:
        c, s, z = outs[i % R]
        if args.api == "op":
            ops.rotate_quant(xs[i % R], hadamard=w.hadamard, v=v, w_t=wt, prepared=prepared,
                             rank_block=w.rank_block, group=w.group, codes=c, scales=s, zeros=z, dest_rows=dest,
                             rank_mode=mode)
            return
        rc = lib.narhip_rotate_quant(p(xs[i % R]), w.tokens, w.n, w.n, m, q, None, w.k, nb, p(v), p(wt), p(prepared),
                                     None, 0, w.group, p(c), p(s), p(z), None, p(dest), mode, p(ws), ws_bytes,
                                     cstream)
        _lib.check(rc)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / args.steps

    # Roofline of the operator call.  One call is one dispatch sequence on the
    # current stream (full-row rank: proj_mfma -> fold_u -> kron_mfma / rq_seg
    # -> corr_quant; otherwise one rq_seg / kron dispatch), so the per-launch
    # duration is ms_step, HIP-event timed above on that stream.  Algorithmic
    # bytes: T*(2n + n/2 + 4n/b) + factor bytes.  Traffic: HBM bytes per call
    # measured with rocprofv3 (FETCH_SIZE x2 + WRITE_SIZE, copy-calibrated).
    t, n, b = w.tokens, w.n, w.group
    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / (ms_step * 1e-3) / 1e9
    kron = w.hadamard[0] > 1
    if full_row_rank and mode != ops.RANK_EXACT and (w.k >= 16 or mode == ops.RANK_MFMA):
        kernels = f"proj_mfma + fold_u + {'kron_mfma' if kron else 'rq_seg'} + corr_quant"
    elif full_row_rank and mode == ops.RANK_AUTO and not kron:
        kernels = "proj_f64 + fold_f64 + rq_seg"
    elif full_row_rank:
        kernels = "proj_exact + corr_exact + rq_row" if kron else "proj_exact + rq_seg"
    else:
        kernels = "kron_mfma" if kron else "rq_seg"
    sha = sources_sha256()
    traffic, traffic_status = measured_traffic(args.config, sha) if mode == ops.RANK_AUTO else (None, "auto only")
    line = {
        "metric": METRIC,
        "value": t / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, narhip/workloads.py)",
        "config": {"workload": describe(w), "tokens": t, "n": n, "hadamard": list(w.hadamard), "k": w.k,
                   "group": b, "rank_mode": args.rank_mode, "rotated_buffers": R},
        "achieved_gbps": alg_bytes / (ms_step * 1e-3) / 1e9,
        "hbm_frac": alg_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "wall_s": wall,
        "roofline": {"kernel": f"rotate_quant call ({kernels})", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": traffic, "traffic_source": "profiles/hbm_traffic.md" if traffic else None,
                     "traffic_status": traffic_status},
        "kernel_sources_sha256": sha,
        "api": args.api,
    }
    busy = measured_mfma_busy(args.config, sha) if mode == ops.RANK_AUTO else None
    if busy:
        line["rank_stage_mfma_busy"] = dict(busy, source="profiles/mfma_utilisation.md")
    if w.dest_rows is not None:
        line["us_per_call"] = ms_step * 1e3
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


def bench_transform_f16(args, w, dev) -> int:
    """E28's NARDownTransform step: fp16 [T, n] -> fp16, H_128 blocks minus (x Y') W''^T."""
    import numpy as np
    import torch

    from narhip import ops
    x_host = torch.from_numpy(w.x.view(np.int16))
    R = max(2, min(8, -(-2 * MALL_BYTES // max(w.x.nbytes, 1)) + 1))
    xs = [x_host.to(dev).view(torch.float16) for _ in range(R)]
    outs = [torch.empty_like(xs[0]) for _ in range(R)]
    v = torch.from_numpy(w.v).to(dev)
    wt = torch.from_numpy(w.w_t).to(dev)

    from narhip import _lib
    lib = _lib.load()
    T, n, k = w.tokens, w.n, w.k
    ws_bytes = lib.narhip_transform_f16_workspace(T, n, k)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    cs = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def step(i: int) -> None:
        if args.api == "op":
            ops.transform_f16(xs[i % R], wt, v=v, had_q=128, out=outs[i % R])
            return
        _lib.check(lib.narhip_transform_f16(p(xs[i % R]), T, n, n, 128, p(v), None, 0, p(wt), k, p(outs[i % R]),
                                            p(ws), ws_bytes, cs))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    t, n = w.tokens, w.n
    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / (ms_step * 1e-3) / 1e9
    from narhip.build import sources_sha256
    sha = sources_sha256()
    traffic, traffic_status = measured_traffic(f"{args.config}_{t}", sha)
    line = {
        "metric": "E28 fp16 down_proj transform (NARDownTransform.forward): tokens/s, 1 MI355X",
        "value": t / (ms_step * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "us_per_call": ms_step * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded, narhip/workloads.py)",
        "config": {"workload": f"{w.name}: {t} tokens x {n} fp16, H128 per block, k={w.k}, fp16 out",
                   "tokens": t, "n": n, "k": w.k, "rotated_buffers": R},
        "achieved_gbps": achieved, "hbm_frac": achieved / HBM_PEAK_GBPS, "wall_s": wall,
        "roofline": {"kernel": "transform_f16 call (proj_tok + xform128)", "bound": "hbm",
                     "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "traffic_source": "profiles/hbm_traffic.md" if traffic else None,
                     "traffic_status": traffic_status},
        "kernel_sources_sha256": sha,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_transform(w, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


def bench_hook(args, dev) -> int:
    """The fused hook call (rotate, dynamic_asym_int4, dequantize; one kernel) through the C ABI:
    hook_kcache_3b -- the K-cache shape (2048 x 8 heads x 128 bf16, H_128 and rank 2 per head, b = 32);
    hook_rows_8192 -- 4096 rows of 8192 bf16 (full-row FWHT, the Llama-3.2-3B down_proj width, b = 128);
    hook_rows_qwen3_8b -- 2048 rows of 9728 bf16 (H_76 x H_128, the Qwen3-8B down_proj width, b = 128:
    the whole-row Paley kernel, x' staged in a workspace, then the quantizer)."""
    import numpy as np
    import torch

    from narhip import _lib, workloads
    if args.config == "hook_kcache_3b":
        w = workloads.kcache_3b(args.tokens or 2048)
        m, q, nb = 1, 128, 128
        desc = f"hook_kcache_3b: {w.tokens} x 8 heads x 128 bf16, H128 + rank 2 per head, b=32, tuple out"
    elif args.config == "hook_rows_qwen3_8b":
        T, n = args.tokens or 2048, 9728
        rng = np.random.default_rng(20260902)
        x = rng.standard_normal((T, n), dtype=np.float32)
        w = workloads.Workload("hook_rows_qwen3_8b", workloads.bf16_bits(x), (76, 128), 128)
        m, q, nb = 76, 128, n
        desc = f"hook_rows_qwen3_8b: {T} x {n} bf16, H76 (Paley II) x H128 whole rows, b=128, tuple out"
    else:
        T, n = args.tokens or 4096, 8192
        rng = np.random.default_rng(20260902)
        x = rng.standard_normal((T, n), dtype=np.float32)
        w = workloads.Workload("hook_rows_8192", workloads.bf16_bits(x), (1, n), 128)
        m, q, nb = 1, n, n
        desc = f"hook_rows_8192: {T} x {n} bf16, full-row FWHT, b=128, tuple out"
    T, n, b = w.tokens, w.n, w.group
    k = w.k
    x = torch.from_numpy(w.x.view(np.int16)).to(dev).view(torch.bfloat16)
    v = None if w.v is None else torch.from_numpy(w.v).to(dev)
    wt = None if w.w_t is None else torch.from_numpy(w.w_t).to(dev)
    codes = torch.empty((T, n), dtype=torch.uint8, device=dev)
    sc = torch.empty((T, n // b), dtype=torch.float16, device=dev)
    zc = torch.empty((T, n // b), dtype=torch.float16, device=dev)
    deq = torch.empty((T, n), dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws_bytes = lib.narhip_rotate_dynamic_asym_int4_workspace(T, n, m, q, k, nb, b, 0)
    assert ws_bytes == 0 or m > 28, "the fused hook shapes run in one kernel"
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    cs = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def step():
        _lib.check(lib.narhip_rotate_dynamic_asym_int4(p(x), T, n, n, m, q, None, k, nb, p(v), p(wt), b, p(codes),
                                                       p(sc), p(zc), p(deq), 0, p(ws) if ws_bytes else None,
                                                       ws_bytes, cs))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / args.steps
    # x read once, codes (one byte each), fp32 deq and fp16 scale / zero written, factors read once
    alg = T * (2 * n + n + 4 * n + 4 * n // b) + (0 if v is None else v.numel() * 4 + wt.numel() * 4)
    achieved = alg / (ms * 1e-3) / 1e9
    from narhip.build import sources_sha256
    sha = sources_sha256()
    traffic, status = measured_traffic(args.config, sha)
    line = {
        "metric": "fused rotate -> dynamic_asym_int4 hook (tuple out): tokens/s, 1 MI355X",
        "value": T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "us_per_call": ms * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded)",
        "config": {"workload": desc, "tokens": T, "n": n, "group": b},
        "roofline": {"kernel": "rotate_dynamic_asym_int4 (one kernel)", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "traffic_status": status},
        "kernel_sources_sha256": sha,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_w4a4(args, dev) -> int:
    """Group-asymmetric W4A4 GEMM on the Llama-3.1-8B down_proj shape: packed INT4
    activations [T, 14336] x packed INT4 weights [4096, 14336], fp32 out."""
    import numpy as np
    import torch

    from narhip import ops
    T, n, O = args.tokens or 8192, 14336, 4096
    rng = np.random.default_rng(20260902)
    f16 = lambda x: torch.from_numpy(np.asarray(x, np.float16)).to(dev)  # noqa: E731
    a = torch.from_numpy(rng.integers(0, 256, (T, n // 2), dtype=np.uint8)).to(dev)
    w = torch.from_numpy(rng.integers(0, 256, (O, n // 2), dtype=np.uint8)).to(dev)
    sa, za = f16(rng.uniform(0.005, 0.2, (T, n // 128))), f16(rng.uniform(-2, 1, (T, n // 128)))
    sw, zw = f16(rng.uniform(0.001, 0.02, (O, n // 128))), f16(rng.uniform(-0.1, 0.05, (O, n // 128)))
    out = torch.empty((T, O), dtype=torch.float32, device=dev)

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / steps

    ms = timed(lambda: ops.w4a4_gemm(a, sa, za, w, sw, zw, out=out), args.steps, args.warmup)
    xb = torch.randn((T, n), device=dev, dtype=torch.bfloat16)
    wb = torch.randn((n, O), device=dev, dtype=torch.bfloat16)
    ms_bf16 = timed(lambda: torch.mm(xb, wb), args.steps, args.warmup)
    ops_per = 2.0 * T * O * n
    achieved = ops_per / (ms * 1e-3) / 1e12
    line = {
        "metric": "group-asymmetric W4A4 GEMM (packed INT4 A and W, fp16 scale/zero per 128): tokens/s, 1 MI355X",
        "value": T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8 (e4m3 INT4 codes)",
        "data": "synthetic (seeded codes and scales)",
        "config": {"workload": f"w4a4_8b: {T} x {n} INT4 activations, {O} x {n} INT4 weights, b=128, fp32 out",
                   "tokens": T, "n": n, "out_features": O},
        "roofline": {"kernel": "w4a4_kernel", "bound": "mfma", "achieved": achieved, "peak": 5000.0,
                     "unit": "TOPS", "frac": achieved / 5000.0, "traffic": None},
        "torch_bf16_mm_ms": ms_bf16,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_transform(w, target_s: float) -> dict:
    """reference_transform (quarot-llama3/nar_r4_kernel.py:190-202) on the host cores."""
    import numpy as np
    import torch

    import nar_r4_kernel as nk
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    y, wt = torch.from_numpy(w.v), torch.from_numpy(w.w_t)
    x = torch.from_numpy(w.x.view(np.float16))

    def once(r: int) -> float:
        t0 = time.perf_counter()
        nk.reference_transform(x[:r], y, wt).half()
        return time.perf_counter() - t0

    rows = min(w.tokens, 16)
    once(rows)
    dt = once(rows)
    while dt * 6 < target_s and rows < w.tokens:
        rows = min(w.tokens, rows * 2)
        dt = once(rows)
    med = statistics.median([once(rows) for _ in range(5)])
    return {"value": rows / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {rows} of {w.tokens} rows, reference_transform in torch fp32 on the CPU, "
                      "median of 5 after 1 warmup"}


if __name__ == "__main__":
    sys.exit(main())
