#!/usr/bin/env python
"""Headline benchmark: packed decode attention on one MI355X (BASELINE config 2 by default).

    python bench.py [--steps K] [--warmup W] [--config 2|3|4|5] [--configs 3,4,5|none]
                    [--cpu-baseline on|off]

A step is one decode-attention call (rotate q, split-K page scan, merge + output
rotation) over the whole batch, one new query token per sequence, with the
packed pages already resident in HBM. Several identical copies of the page pool
are rotated between steps so the 256 MB Infinity Cache cannot serve repeats.
Prints ONE JSON line on stdout; details go to stderr.

``value`` is decode tokens/s = B / step time (whole job, one GPU).
``roofline.achieved`` is the algorithmic KV bytes of one step
(sum_b L_b * Hkv * ((NB_K + 2) + (NB_V + 2)), the reference's traffic model,
bench_packed_attention.py:91-98) divided by the mean duration of the page-scan
kernel, timed with HIP events recorded on its stream around every launch.
``roofline.traffic`` is the HBM bytes one scan launch moves, read from the
FETCH_SIZE and WRITE_SIZE counters of two ``rocprofv3 --pmc`` child runs and
scaled by what the same counters read for a 1 GiB device copy.
``cpu_baseline`` times the CPU restatement of the reference's CPU decode path
(``tiled_compressed_attention``) on a bounded sample of page-table columns of
the same workload and scales it to the full step.
``configs`` repeats the decode measurement (scan time, its fraction of 8 TB/s,
tokens/s, sampled parity against the oracle) for the other BASELINE configs.
``lds_floor`` is the scan's LDS ceiling: its codebook lookups are 8-byte LDS
reads at data-dependent addresses, head_dim wave-level reads per 64-token chunk of
a kv head, and the LDS of a CU serves them at a rate the probe
``wn_probe_lds_lookup_rate`` measures in the same run (eight waves per CU, as the
scan runs); ``floor_us`` is the time those reads alone need, ``scan_over_floor``
the scan's time against it. The scan's other LDS traffic (its score tile and p
words) comes on top.
``prefill`` times the fused prefill over the packed pages (Q = 16 new tokens per
sequence, and Q = 512 for two sequences) beside the reference's Q > 1 route on the same
pages and GPU (dequantize each history, then SDPA), with the scan's HBM and MFMA
fractions and sampled parity against the oracle.
``allow_tf32`` times the reference's ``allow_tf32=True`` decode on the same pages
(the TF32-class scan: single fp16 operands, fp32 accumulation) with its own sampled
parity; the headline line stays the default, fp32-exact decode.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode-attn tokens/s + HBM GB/s (% peak), 4-bit packed KV, 32k ctx, 1 GPU"
HBM_PEAK_GBPS = 8000.0

sys.path.insert(0, str(ROOT / "tests"))
import workloads  # noqa: E402  (shared with the full-size GPU parity tests)

CONFIGS = workloads.CONFIGS
DATA_NOTE = ("synthetic, seeded: lengths, page order, outlier channels, head scales and q from "
             "torch.Generator().manual_seed(config seed); K/V drawn on the GPU from a generator seeded "
             "with the same seed (a CPU draw of the 1e9-4.4e9 normals takes minutes), cast to bf16 and "
             "packed by the product append kernel; q ~N(0,1) bf16")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def scan_kernel_name(c) -> str:
    """Symbol of the page-scan kernel wn_decode_attention launches for this shape."""
    scan = os.environ.get("WN_DECODE_SCAN", "rows") or "rows"
    n_rep = c["Hq"] // c["Hkv"]
    fits = n_rep <= 8 or (n_rep <= 16 and n_rep % 2 == 0)   # even n_rep > 8: two virtual heads per kv head
    if c["D"] == 128 and fits and c["S"] >= 16 and scan != "valu":
        pair = (c["bwk"], c["bwv"])
        fp16_split = (pair[0] == pair[1] and pair[0] in (2, 3, 4, 5, 6)) or pair in ((4, 6), (6, 4))
        return "decode_rows16_kernel" if fp16_split and scan != "rows32" else "decode_rows_kernel"
    return "decode_split_kernel"


def tf_kernel_name(c) -> str:
    """Symbol of the page-scan kernel wn_decode_attention_tf32 launches for this shape:
    the TF32-class row scan for 4 and 6-bit K and V on the row scan, else the default's."""
    if (scan_kernel_name(c) == "decode_rows16_kernel" and c["bwk"] in (4, 6) and c["bwv"] in (4, 6)):
        return "decode_rows_tf_kernel"
    return scan_kernel_name(c)


def prefill_kernel_name(n_rep: int, Q: int) -> str:
    """Symbol of the prefill scan wn_prefill_attention launches: the shared-tile scan
    once a kv head has eight 32-row query blocks (n_rep * Q rounded up to 64 rows,
    at least 256), else the per-wave scan."""
    rows = (n_rep * Q + 63) // 64 * 64
    return "pf_tile_kernel" if rows // 32 >= 8 else "pf_scan_kernel"


kv_bytes = workloads.kv_bytes


def copy_peak(dev, nbytes: int = 1 << 30, reps: int = 10):
    """Device-to-device copy of ``nbytes`` (torch's copy kernel): GB/s of read + write bytes.

    Gives the measured bandwidth ceiling on this box beside the 8 TB/s data-sheet
    peak, and a plain copy kernel of known size for scaling the FETCH_SIZE /
    WRITE_SIZE counters of a profiling run.
    """
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / reps * 1e-3
    del src, dst
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": t * 1e6, "GBps": 2 * nbytes / t / 1e9}


def hbm_traffic(cfg: int, kernel: str, timeout_s: int = 120, tf32: bool = False):
    """HBM bytes one launch of ``kernel`` moves, from two ``rocprofv3 --pmc`` child runs.

    Each pass profiles a short run of this script (3 steps plus the 1 GiB device
    copy of ``copy_peak``) with one counter, FETCH_SIZE then WRITE_SIZE (KiB per
    dispatch). Each counter is scaled by what it reads for that copy of known size
    (bytes / counter), so the figure is in real bytes whatever fraction of the
    memory channels the counter samples. Returns None when the profiler is absent
    or a pass fails; the bench line then carries ``traffic: null``. ``tf32`` profiles
    the allow_tf32 leg of the child run instead of its default decode.
    """
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if not prof:
        return None
    out = {}
    with tempfile.TemporaryDirectory(prefix="wn_pmc_", dir="/tmp") as tmp:
        env = dict(os.environ, TMPDIR="/tmp")
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = Path(tmp) / counter
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", str(d), "-o", "run", "--",
                   sys.executable, str(ROOT / "bench.py"), "--config", str(cfg), "--steps", "3", "--warmup", "1",
                   "--settle", "0", "--parity", "off", "--cpu-baseline", "off", "--traffic", "off", "--append", "off",
                   "--configs", "none", "--tf32", "on" if tf32 else "off", "--config-steps", "3",
                   "--dequant", "off", "--dense", "off",
                   "--copy-peak", "on"]
            try:
                subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                               timeout=timeout_s, check=True)
            except (subprocess.SubprocessError, OSError) as e:
                log(f"traffic pass {counter} failed: {e}")
                return None
            files = list(d.rglob("*counter_collection.csv"))
            if not files:
                return None
            scan, copy = [], []
            for r in csv.DictReader(open(files[0])):
                v = float(r["Counter_Value"])
                if kernel in r["Kernel_Name"]:
                    scan.append(v)
                elif "copyBuffer" in r["Kernel_Name"]:
                    copy.append(v)
            # the 13 copies of copy_peak move 1 GiB each, more than any other copy of the run
            copy = sorted(copy)[-10:]
            if not scan or len(copy) < 10:
                return None
            copy_kib = statistics.median(copy)
            factor = (1 << 30) / (copy_kib * 1024)
            out[counter] = {"kib_per_launch": statistics.fmean(scan), "copy_kib": copy_kib, "factor": factor,
                            "bytes_per_launch": statistics.fmean(scan) * 1024 * factor}
    out["bytes_per_launch"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
    return out


def dense_bench(c, lens, q, dev, steps: int = 30, warmup: int = 5, copies: int = 2, check_len: int = 2048):
    """The matched unquantized baseline (dense_decode_attention, packed_attention_triton.py:190-201;
    the reference's ``dense_paged`` arm, bench_packed_attention.py:101-117) at the same
    batch, heads, lengths, page size and query: bf16 pages (P, Hkv, S, D), ~N(0, 1),
    contiguous tables, ``copies`` pools rotated between steps as for the packed step.

    Bytes per step: sum(L) * Hkv * 2 * D * 2 (K and V rows, the reference's dense
    traffic model, bench_packed_attention.py:99). The scan kernel is timed with HIP
    events on its stream, the step with events around the calls. Parity: two
    sequences cut to ``check_len`` tokens against the float64 oracle on the same pages.
    """
    import torch
    from oracle import attention as oa
    from winnow_amd import packed_attention as pa

    B, Hkv, D, S = len(lens), c["Hkv"], c["D"], c["S"]
    need = [(L + S - 1) // S for L in lens]
    P = sum(need)
    table = torch.full((B, max(need)), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        table[b, :need[b]] = torch.arange(off, off + need[b], dtype=torch.int32)
        off += need[b]
    dtable, dl = table.to(dev), torch.tensor(lens, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(99)
    kvs = []
    for _ in range(copies):
        kp = torch.randn(P, Hkv, S, D, generator=g, device=dev, dtype=torch.bfloat16)
        vp = torch.randn(P, Hkv, S, D, generator=g, device=dev, dtype=torch.bfloat16)
        kvs.append(pa.DenseKV(kp, vp, dtable, dl, D))
    scale = 1.0 / math.sqrt(D)
    pps, ns = pa.dense_plan_for(q, kvs[0])
    ws = torch.empty(pa.workspace_bytes(B, q.shape[1], Hkv, D, pps, ns), dtype=torch.uint8, device=dev)
    for i in range(warmup):
        pa.dense_decode_attention(q, kvs[i % copies], scale, workspace=ws, check_ranges=False)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record()
        e1.record()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        e0, e1 = evs[i]
        pa.dense_decode_attention(q, kvs[i % copies], scale, workspace=ws, check_ranges=False,
                                  timing_events=(ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event)))
    end.record()
    torch.cuda.synchronize()
    kern_ms = statistics.fmean(e0.elapsed_time(e1) for e0, e1 in evs)
    # the step time without the per-launch events (as measure_decode)
    start.record()
    for i in range(steps):
        pa.dense_decode_attention(q, kvs[i % copies], scale, workspace=ws, check_ranges=False)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    nbytes = sum(lens) * Hkv * 2 * D * 2
    # parity on two sequences cut to check_len tokens (same pages, shorter seq_lens)
    seqs = [0, B - 1]
    cut = torch.tensor([min(check_len, lens[b]) for b in seqs], dtype=torch.int32)
    kv0 = kvs[0]
    sub = pa.DenseKV(kv0.k_pages, kv0.v_pages, dtable[seqs], cut.to(dev), D)
    got = pa.dense_decode_attention(q[seqs], sub, scale, out_dtype=torch.float32).cpu()
    used = torch.unique(table[seqs, :(check_len + S - 1) // S].flatten()).long()
    kpc = torch.zeros(P, Hkv, S, D, dtype=torch.bfloat16)
    vpc = torch.zeros(P, Hkv, S, D, dtype=torch.bfloat16)
    kpc[used], vpc[used] = kv0.k_pages[used.to(dev)].cpu(), kv0.v_pages[used.to(dev)].cpu()
    ref = oa.dense_paged_attention_f64(q[seqs].float().cpu(), kpc, vpc, table[seqs], cut, scale)
    err = (got.double() - ref).abs().max().item()
    del kvs, ws
    torch.cuda.empty_cache()
    return {"us_per_step": ms * 1e3, "scan_kernel_us": kern_ms * 1e3, "bytes_per_step": nbytes,
            "scan_GBps": nbytes / (kern_ms * 1e-3) / 1e9, "scan_frac_of_8TBps": nbytes / (kern_ms * 1e-3) / 8e12,
            "tokens_per_s": B / (ms * 1e-3), "page_dtype": "bf16", "splits": ns, "pages_per_split": pps,
            "parity_max_abs_err_vs_f64": err, "parity_within_2e-3_1e-3": bool(
                torch.allclose(got.double(), ref, atol=2e-3, rtol=1e-3))}


def append_bench(c, lens, table, quants, dev, reps: int = 200, n_new: int = 16):
    """The append path of ``PagedPackedCache.update`` (packed_backend.py:136-170): quantize,
    pack and scatter ``n_new`` new tokens per sequence, K and V, at positions
    L_b .. L_b + n_new - 1, timed separately from attention.

    The new tokens go to one fresh page per sequence, addressed through the
    sequence's page-table column L_b / S as in the cache; they land in a small
    separate pool so the decode pool is left as it is. Timed with hipEvents over
    events the library records around the kernel on each of ``reps`` calls (and, as
    ``us_per_call_from_python``, over ``reps`` back-to-back calls of the Python wrapper,
    whose host overhead is longer than the kernel; as ``us_per_call_from_python_plan``,
    the same through the ``AppendPlan`` the cache keeps per layer; as ``us_per_call_graph``, over replays
    of a HIP graph of back-to-back calls, the GPU time per call of a serving loop that
    captures its appends); checked against the CPU
    restatement (codes under the adjudication protocol) and timed beside it.
    """
    import torch
    sys.path.insert(0, str(ROOT / "tests"))
    from adjudicate import adjudicate_codes
    from oracle import append as oapp
    from oracle import packing as opk
    from oracle.quantizer import get_quantizer as oq
    from winnow_amd import packed_backend as pb
    from winnow_amd.packing import packed_bytes

    B, Hkv, D, S = len(lens), c["Hkv"], c["D"], c["S"]
    kq, vq = quants
    nbk, nbv = packed_bytes(D, c["bwk"]), packed_bytes(D, c["bwv"])
    g = torch.Generator().manual_seed(c["seed"] + 100)
    k = torch.randn(B, Hkv, n_new, D, generator=g).bfloat16()
    v = torch.randn(B, Hkv, n_new, D, generator=g).bfloat16()
    start = torch.tensor(lens, dtype=torch.int32)
    width = max((L + n_new + S - 1) // S for L in lens)
    tab = torch.full((B, width), -1, dtype=torch.int32)
    P = 0
    for b, L in enumerate(lens):                 # fresh pages for the new tokens' columns
        for col in range(L // S, (L + n_new + S - 1) // S):
            tab[b, col] = P
            P += 1
    kp = torch.zeros(P, Hkv, S, nbk, dtype=torch.uint8, device=dev)
    vp = torch.zeros(P, Hkv, S, nbv, dtype=torch.uint8, device=dev)
    kn = torch.zeros(P, Hkv, S, dtype=torch.float16, device=dev)
    vn = torch.zeros(P, Hkv, S, dtype=torch.float16, device=dev)
    kd, vd, td, sd = k.to(dev), v.to(dev), tab.to(dev), start.to(dev)

    def call(check=False, evs=None):
        pb.append_kv(kd, vd, kq, vq, kp, vp, kn, vn, td, sd, check_ranges=check, timing_events=evs)

    call(check=True)                             # full validation once, outside the timed region
    for _ in range(20):
        call()
    # kernel time: events the library records on the stream right around the kernel
    # (the Python wrapper's host overhead per call is longer than the kernel)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in evs:                           # torch's "recorded" flag; the library records them again
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    for e0, e1 in evs:
        call(evs=(ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event)))
    torch.cuda.synchronize()
    us = statistics.fmean(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3
    # the same calls back to back from Python, host overhead included
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    host_us = e0.elapsed_time(e1) / reps * 1e3
    # the same through an AppendPlan, as PagedPackedCache.update appends a layer: the
    # pages, norms and quantizers checked once, each call checking the step's operands
    plan = pb.AppendPlan(kq, vq, kp, vp, kn, vn)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        plan.launch(plan.bind(kd, vd, td, sd))
    e1.record()
    torch.cuda.synchronize()
    plan_us = e0.elapsed_time(e1) / reps * 1e3
    # back to back on the GPU with neither events nor Python between the calls: 32 calls
    # captured in one HIP graph (no memsets or allocations inside), replayed; the byte
    # check below reads the pages the replays wrote last
    graph_calls, graph_reps = 32, 20
    graph_us = None
    try:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(graph_calls):
                call()
        gr.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(graph_reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        graph_us = e0.elapsed_time(e1) / (graph_reps * graph_calls) * 1e3
    except RuntimeError as exc:                  # capture refused: report the other two timings
        print(f"append graph timing skipped: {exc}", file=sys.stderr, flush=True)

    # CPU restatement on the same inputs, timed, then the byte check
    ref = [torch.zeros(P, Hkv, S, nb, dtype=torch.uint8) for nb in (nbk, nbv)]
    refn = [torch.zeros(P, Hkv, S, dtype=torch.float16) for _ in range(2)]
    okq, ovq = oq(c["bwk"], D, 42), oq(c["bwv"], D, 42)
    t0 = time.perf_counter()
    oapp.append(k, okq, ref[0], refn[0], tab, lens)
    oapp.append(v, ovq, ref[1], refn[1], tab, lens)
    cpu_us = (time.perf_counter() - t0) * 1e6
    flips = 0
    for src, got, want, bw, tq in ((k, kp, ref[0], c["bwk"], okq), (v, vp, ref[1], c["bwv"], ovq)):
        gc = torch.from_numpy(opk.unpack(got.cpu().numpy(), bw, D))
        wc = torch.from_numpy(opk.unpack(want.numpy(), bw, D))
        pos = torch.tensor([[L + i for i in range(n_new)] for L in lens])
        pids = torch.gather(tab.long(), 1, pos // S)
        sel = lambda t: t[pids, :, pos % S].permute(0, 2, 1, 3)      # noqa: E731
        flips += adjudicate_codes(src, sel(gc), sel(wc), tq)
    vectors = 2 * B * Hkv * n_new
    return {"us_per_call": us, "timing": "kernel, hipEvents recorded by wn_append_kv around its launch",
            "us_per_call_from_python": host_us, "us_per_call_from_python_plan": plan_us,
            "us_per_call_graph": graph_us,
            "graph": f"{graph_calls} calls per HIP graph, {graph_reps} replays between one event pair",
            "vectors_per_call": vectors, "vectors_per_s": vectors / (us * 1e-6),
            "new_tokens_per_seq": n_new, "bytes_read": 2 * B * Hkv * n_new * D * 2,
            "bytes_written": B * Hkv * n_new * (nbk + 2 + nbv + 2),
            "cpu_us_per_call": cpu_us, "cpu_kind": "port", "adjudicated_code_flips": flips,
            "codes_checked": vectors * D}


# The reference's retained RTX A6000 numbers at N = 1,048,576, D 128 (µs per call): its
# TF32 Triton arm (allow_tf32=True, the class of this build's fast mode), its fp32
# arms (the numeric peers of this build's default mode: the fp32 Triton kernel at 4
# bits, the exact CUDA kernel at 6 bits) and torch's eager reference.
REF_DEQUANT_A6000 = {
    4: {"tf32_triton_us": 1301.9, "fp32_triton_us": 108269.1, "torch_us": 8542.6,
        "source": "results/phaseC_kernel_tf32.json rows[23], results/phaseC_kernel.json rows[23]"},
    6: {"tf32_triton_us": 1299.0, "cuda_exact_us": 10548.3, "torch_us": 44768.4,
        "source": "results/phaseC_kernel_bw6.json rows[23], turboquant_kv/README.md:335-337"},
}


def dequant_bench(dev, bws=(4, 6), reps: int = 50, check_rows: int = 2048, cpu_rows: int = 32768,
                  fast: bool = False):
    """The fused history dequantization (``wn_tq_dequant``) at the shape the reference
    publishes its dequant numbers for: N = 1,048,576 vectors (B16 x H4 x L16384), D 128,
    bf16 out (``turboquant_kv/README.md:203-204``, ``results/phaseC_kernel_tf32.json``).

    Random packed bytes are valid codes at every width. Bytes per vector: NB packed +
    2 norm read, 2 D written. Timed with hipEvents over ``reps`` calls; the first
    ``check_rows`` / 2 and the last ``check_rows`` / 2 rows are checked against the float64 closed form, and the CPU
    restatement (torch fp32 ``centroids[idx] @ Pi * n``) is timed on ``cpu_rows`` rows
    and scaled to N.
    """
    import torch
    from oracle import packing as opk
    from winnow_amd.kernel import tq_dequant
    from winnow_amd.packing import packed_bytes
    from winnow_amd.quantizer import get_quantizer

    B, H, L, D = 16, 4, 16384, 128
    N = B * H * L
    res = {}
    for bw in bws:
        nb = packed_bytes(D, bw)
        tq = get_quantizer(bw, D, dev, 42)
        g = torch.Generator(device=dev).manual_seed(bw)
        packed = torch.randint(0, 256, (B, H, L, nb), dtype=torch.uint8, device=dev, generator=g)
        norms = (torch.rand(B, H, L, device=dev, generator=g) * 20 + 1).half()
        out = torch.empty(B, H, L, D, dtype=torch.bfloat16, device=dev)

        def call():
            tq_dequant(packed, norms, tq.centroids, tq.Pi, bw, D, out=out, allow_tf32=fast)

        for _ in range(5):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        moved = N * (nb + 2 + 2 * D)
        # float64 check of the first and the last rows (the first and the last pass of
        # every wave's pipeline)
        rows = torch.cat([torch.arange(check_rows // 2), torch.arange(N - check_rows // 2, N)]).to(dev)
        pc = packed.view(N, nb)[rows].cpu().numpy()
        idx = torch.from_numpy(opk.unpack(pc, bw, D)).long()
        c64, pi64 = tq.centroids.cpu().double(), tq.Pi.cpu().double()
        ref = (c64[idx] @ pi64) * norms.view(N)[rows].cpu().double()[:, None]
        got = out.view(N, D)[rows].cpu().double()
        err = (got - ref).abs().max().item()
        ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
        ok = bool(((got - ref).abs() <= ulp + (2e-3 if fast else 2e-5) * ref.abs().max()).all())
        # CPU restatement, bounded sample
        c32, pi32 = tq.centroids.cpu(), tq.Pi.cpu()
        pcs = torch.from_numpy(opk.unpack(packed.view(N, nb)[:cpu_rows].cpu().numpy(), bw, D)).long()
        ns = norms.view(N)[:cpu_rows].cpu().float()
        _ = ((c32[pcs[:1024]] @ pi32) * ns[:1024, None]).bfloat16()  # untimed: first-call set-up
        t0 = time.perf_counter()
        _ = ((c32[pcs] @ pi32) * ns[:, None]).bfloat16()
        cpu_us = (time.perf_counter() - t0) * 1e6 * N / cpu_rows
        res[f"{bw}bit" + ("_allow_tf32" if fast else "")] = {"us_per_call": us, "vectors": N, "GBps": moved / (us * 1e-6) / 1e9,
                           "frac_of_8TBps": moved / (us * 1e-6) / 8e12, "bytes_per_call": moved,
                           "max_abs_err_vs_f64": err, "within_bf16_step": ok,
                           "cpu_us_per_call": cpu_us, "cpu_sample_rows": cpu_rows, "cpu_threads": torch.get_num_threads(),
                           "reference_a6000": REF_DEQUANT_A6000.get(bw)}
    return res


def parity(w, kv=None, seqs=None, allow_tf32: bool = False):
    """Same-run checks on the same pages: the first, middle and last sequences' attention
    against the CPU oracle (2e-3 max-abs / 1e-3 relative of the fp32 output) and the
    float64 oracle (relative L2), and sequence 0's first 256 tokens re-quantized by the
    oracle against the pool bytes (adjudicated flips). ``allow_tf32`` checks the
    TF32-class decode instead of the default one."""
    import torch
    from cases import to_host
    from oracle import attention as oa
    from winnow_amd import packed_attention as pa

    kv = kv or w.kvs[0]
    B = len(w.lens)
    seqs = seqs or sorted({0, B // 2, B - 1})
    scale = oa.default_scale(w.c["D"])
    got = pa.packed_decode_attention(w.q, kv, scale, out_dtype=torch.float32, allow_tf32=allow_tf32).cpu()[seqs]
    sub = to_host(kv, seqs)
    qs = w.q.float().cpu()[seqs]
    ref = oa.tiled_compressed_attention(qs, sub, scale)
    f64 = oa.reconstruct_attention_f64(qs, sub, scale)
    rq = workloads.requantize(w, kv)
    tf = {}
    if allow_tf32:
        # also against the float64 decode of operands rounded as the TF32-class scan rounds them
        from tf32_reference import tf32_class_reference
        rr = tf32_class_reference(qs, sub, scale).float()
        tf = {"rounded_operand_ref_max_abs_err": (got - rr).abs().max().item(),
              "rounded_operand_ref_within_2e-3_1e-3": bool(torch.allclose(got, rr, atol=2e-3, rtol=1e-3))}
    return {"sequences": seqs, **tf, "attn_max_abs_err": (got - ref).abs().max().item(),
            "attn_within_2e-3_1e-3": bool(torch.allclose(got, ref, atol=2e-3, rtol=1e-3)),
            "rel_l2_vs_f64": ((got.double() - f64).norm() / f64.norm()).item(),
            "requantized": f"sequence 0 (all {w.sample[0].shape[2]} tokens) and {rq['random_pages']} random "
                           "pages of three other sequences, K and V",
            "codes_checked": rq["vectors"] * w.c["D"], "adjudicated_code_flips": rq["code_flips"],
            "norms_checked": rq["vectors"], "adjudicated_norm_flips": rq["norm_flips"]}


def cpu_model() -> str:
    """The host CPU's model name (``lscpu``'s "Model name", read from /proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def measure_decode(w, steps: int, warmup: int, settle: float, splits=None, allow_tf32: bool = False):
    """Time ``steps`` decode steps of workload ``w`` (pools rotated between steps): the
    page-scan kernel from HIP events the C ABI records on its stream around every
    launch, then the step time from events around the same number of calls with
    nothing recorded between them. ``allow_tf32`` times the TF32-class decode
    (``wn_decode_attention_tf32``)."""
    import torch
    from winnow_amd import packed_attention as pa

    q, kvs = w.q, w.kvs
    B, Hq, Hkv, D = len(w.lens), w.c["Hq"], w.c["Hkv"], w.c["D"]
    scale = 1.0 / math.sqrt(D)
    pps, ns = pa.plan_for(q, kvs[0], splits, allow_tf32)
    ws = torch.empty(pa.workspace_bytes(B, Hq, Hkv, D, pps, ns), dtype=torch.uint8, device=q.device)
    for kv in kvs:
        pa.check_kernel_contract(q, kv)          # full validation once, outside the timed region

    def step(i, evs=None):
        return pa.packed_decode_attention(q, kvs[i % len(kvs)], scale, workspace=ws, check_ranges=False,
                                          timing_events=evs, plan=(pps, ns), allow_tf32=allow_tf32)

    # Bring the GPU to its sustained clocks before the warm-up steps: a few ms of work
    # otherwise times a part-clocked GPU, which a decode server running continuously
    # never sees.
    t_settle = time.perf_counter()
    i = 0
    while time.perf_counter() - t_settle < settle:
        for _ in range(20):
            step(i)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        step(i)
    ev_pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(steps)]
    for e0, e1 in ev_pairs:                       # materialise the underlying hipEvents
        e0.record()
        e1.record()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the scan's duration: events recorded on its stream right around every launch
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        e0, e1 = ev_pairs[i]
        step(i, (ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event)))
    end.record()
    torch.cuda.synchronize()
    kern = [e0.elapsed_time(e1) for e0, e1 in ev_pairs]
    ms_evented = start.elapsed_time(end) / steps
    # the step time: the same steps with nothing between the launches (the events above
    # are extra commands in the stream and lengthen each step by a few microseconds)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    return {"ms_per_step": start.elapsed_time(end) / steps, "ms_per_step_with_scan_events": ms_evented,
            "kernel_ms": statistics.fmean(kern), "kernel_ms_median": statistics.median(kern), "splits": ns,
            "pages_per_split": pps}


def lds_lookup_rate(waves_per_cu: int = 8, iters: int = 8192):
    """Table lookups (8-byte LDS reads at data-dependent addresses, wave instructions)
    one CU's LDS serves per microsecond with ``waves_per_cu`` waves on every CU
    (wn_probe_lds_lookup_rate): the rate the packed row scans' lookups run against."""
    import ctypes
    from winnow_amd import _lib
    r = ctypes.c_double(0.0)
    _lib.probe_call("wn_probe_lds_lookup_rate", waves_per_cu, iters, ctypes.byref(r))
    return r.value


def lds_floor(lens, c, rate, cus):
    """The row scan's LDS floor: it looks codebook entries up in LDS, one 8-byte read
    per two codes, so each 64-token chunk of a kv head costs head_dim wave-level
    lookups (D/2 for K, D/2 for V) whatever its widths and head groups; at ``rate``
    lookups per microsecond per CU the chunks need at least this long."""
    chunks = sum((L + 63) // 64 for L in lens) * c["Hkv"]
    return {"lookups_per_chunk": c["D"], "chunks": chunks, "rate_per_cu_per_us": rate, "cus": cus,
            "floor_us": chunks * c["D"] / (cus * rate)}


def tf32_leg(w, bytes_step: int, steps: int, warmup: int, settle: float, splits, check: bool):
    """The reference's allow_tf32=True decode on the same pages: scan time, fraction of
    8 TB/s, tokens/s and sampled parity (against the oracle's fp32 path at the north-star
    bar)."""
    mt = measure_decode(w, steps, warmup, settle, splits, allow_tf32=True)
    us = mt["kernel_ms"] * 1e3
    return {"kernel": tf_kernel_name(w.c), "scan_us": us, "frac": bytes_step / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "us_per_step": mt["ms_per_step"] * 1e3, "tokens_per_s": len(w.lens) / (mt["ms_per_step"] * 1e-3),
            "step_frac": bytes_step / (mt["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, "steps": steps,
            "products": "single fp16 operands (11 significant bits, rounded to nearest), fp32 accumulation",
            "parity": parity(w, allow_tf32=True) if check else None}


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 matrix-core peak


def _sub_kv(kv, n: int, cut: int | None = None):
    """The first ``n`` sequences of a device PackedKV, lengths optionally cut to ``cut``."""
    from winnow_amd import packed_attention as pa
    lens = kv.seq_lens_host[:n].clone()
    if cut is not None:
        lens = lens.clamp(max=cut)
    return pa.PackedKV(kv.k_pages, kv.k_norms, kv.v_pages, kv.v_norms, kv.page_table[:n],
                       lens.to(kv.seq_lens.device), kv.k_quant, kv.v_quant, kv.head_dim,
                       seq_lens_host=lens, page_table_host=kv.page_table_host[:n])


def _pick(kv, seqs):
    """A device PackedKV restricted to sequences ``seqs`` (same pool)."""
    from winnow_amd import packed_attention as pa
    idx = torch_index(seqs, kv.page_table.device)
    return pa.PackedKV(kv.k_pages, kv.k_norms, kv.v_pages, kv.v_norms, kv.page_table[idx], kv.seq_lens[idx],
                       kv.k_quant, kv.v_quant, kv.head_dim, seq_lens_host=kv.seq_lens_host[list(seqs)],
                       page_table_host=kv.page_table_host[list(seqs)])


def torch_index(seqs, dev):
    import torch
    return torch.tensor(list(seqs), dtype=torch.long, device=dev)


def prefill_bench(w, Q: int, nseq: int | None = None, steps: int = 10, warmup: int = 3, ref_steps: int = 2,
                  check: bool = True, check_len: int = 4096):
    """The fused prefill (``packed_prefill_attention``, wn_prefill_attention) of Q new
    tokens per sequence on the workload's pages, the first ``nseq`` sequences: their
    lengths count the Q tokens (the cache holds them before attention, as on the
    reference's Q > 1 route), query bf16 ~N(0, 1) seeded, output bf16. Beside it the
    reference's route on the same pages and GPU: each history dequantized to bf16, then
    SDPA with the offset causal mask (``_reconstruct_sdpa``, packed_backend.py:211-226).

    The scan is timed with HIP events on its stream; the call (rotate + scan + merge)
    with events around the calls. Its roofline, both ways: HBM, the packed K/V rows and
    norms of each history read once (the decode's algorithmic bytes); MFMA, 4 Hq D flops
    per visible (query, key) pair (query i of a sequence of length L sees L - Q + i + 1
    keys) against the 2.5 PFLOP/s dense fp16 peak. Parity: two sequences cut to
    ``check_len`` tokens against the oracle's fp32 reconstruct_attention."""
    import torch
    from cases import to_host
    from oracle import attention as oa
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    from winnow_amd.packing import packed_bytes

    c = w.c
    kv = _sub_kv(w.kvs[0], nseq or len(w.lens))
    lens = [int(x) for x in kv.seq_lens_host]
    B, Hq, D = len(lens), c["Hq"], c["D"]
    g = torch.Generator(device=w.q.device).manual_seed(1000 + Q)
    q = torch.randn(B, Hq, Q, D, generator=g, device=w.q.device).bfloat16()
    scale = 1.0 / math.sqrt(D)
    ns = pa.prefill_plan_for(q, kv)
    ws = torch.empty(pa.prefill_workspace_bytes(B, Hq, c["Hkv"], Q, D, ns), dtype=torch.uint8, device=q.device)
    call = lambda evs=None: pa.packed_prefill_attention(q, kv, scale, num_splits=ns, workspace=ws,  # noqa: E731
                                                        check_ranges=False, timing_events=evs)
    for _ in range(warmup):
        call()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    for e0, e1 in evs:
        call((ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event)))
    torch.cuda.synchronize()
    scan_ms = statistics.fmean(e0.elapsed_time(e1) for e0, e1 in evs)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        call()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    pb._reconstruct_sdpa(q, kv, scale)
    torch.cuda.synchronize()
    start.record()
    for _ in range(ref_steps):
        pb._reconstruct_sdpa(q, kv, scale)
    end.record()
    torch.cuda.synchronize()
    ref_ms = start.elapsed_time(end) / ref_steps
    nbytes = kv_bytes(lens, c["Hkv"], packed_bytes(D, c["bwk"]), packed_bytes(D, c["bwv"]))
    pairs = sum(max(0, min(L, L - Q + i + 1)) for L in lens for i in range(Q))
    flops = 4 * Hq * D * pairs
    out = {"Q": Q, "batch": B, "q_heads": Hq, "kv_heads": c["Hkv"], "seq_lens": f"{min(lens)}..{max(lens)}",
           "bits_k": c["bwk"], "bits_v": c["bwv"], "splits": ns,
           "kernel": prefill_kernel_name(Hq // c["Hkv"], Q),
           "scan_us": scan_ms * 1e3, "us_per_call": ms * 1e3, "prefill_tokens_per_s": B * Q / (ms * 1e-3),
           "hbm": {"algorithmic_bytes": nbytes, "achieved_GBps": nbytes / (scan_ms * 1e-3) / 1e9,
                   "frac": nbytes / (scan_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS},
           "mfma": {"flops": flops, "achieved_TFLOPs": flops / (scan_ms * 1e-3) / 1e12,
                    "frac": flops / (scan_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS},
           "reference_route": "history dequantized to bf16, then SDPA with the offset causal mask "
                              "(_reconstruct_sdpa, packed_backend.py:211-226)",
           "reference_route_us": ref_ms * 1e3, "speedup_vs_reference_route": ref_ms / ms,
           "products": "single fp16 operands (11 significant bits, rounded to nearest), fp32 accumulation"}
    if check:
        from tf32_reference import prefill_q_log2, tf32_class_reference
        seqs = sorted({0, B - 1})
        sub = _sub_kv(kv, B, cut=check_len)
        qs = q[seqs].contiguous()
        sub2 = _pick(sub, seqs)
        wsc = torch.empty(pa.prefill_workspace_bytes(len(seqs), Hq, c["Hkv"], Q, D, 3), dtype=torch.uint8,
                          device=q.device)
        got = pa.packed_prefill_attention(qs, sub2, scale, num_splits=3, workspace=wsc,
                                          out_dtype=torch.float32).cpu()
        host = to_host(sub2, list(range(len(seqs))))
        ref = oa.reconstruct_attention(qs.float().cpu(), host, scale)
        rr = tf32_class_reference(qs.float().cpu(), host, scale,
                                  q_log2=prefill_q_log2(wsc, len(seqs), Hq, c["Hkv"], Q)).float()
        route = pb._reconstruct_sdpa(qs, sub2, scale).float().cpu()
        out["parity"] = {
            "sequences": seqs, "cut_to": check_len,
            "rounded_operand_ref_max_abs_err": (got - rr).abs().max().item(),
            "rounded_operand_ref_within_2e-3_1e-3": bool(torch.allclose(got, rr, atol=2e-3, rtol=1e-3)),
            "fp32_oracle_max_abs_err": (got - ref).abs().max().item(),
            "fp32_oracle_within_2e-3_1e-3": bool(torch.allclose(got, ref, atol=2e-3, rtol=1e-3)),
            "reference_route_fp32_oracle_max_abs_err": (route - ref).abs().max().item(),
            "note": "the TF32-class operand rounding itself moves this data (1 % outlier channels, 1,024 "
                    "query rows) up to ~4e-3 from the fp32 oracle; the reference's bf16 route moves it more"}
    del ws
    return out


def config_line(cfg: int, dev, steps: int, warmup: int, settle: float, copies: int, check: bool,
                lds_rate: float | None = None, tf32: bool = False, prefill: bool = False):
    """Decode throughput, roofline fraction of the scan and same-run parity at config
    ``cfg``; ``tf32`` adds the allow_tf32 leg on the same pages, ``prefill`` the fused
    prefill of 16 new tokens per sequence."""
    import torch
    from winnow_amd.packing import packed_bytes

    t0 = time.time()
    w = workloads.build(cfg, dev, copies=copies, full_check=check)
    c = w.c
    log(f"config {cfg} built in {time.time() - t0:.1f} s: B={len(w.lens)} sum(L)={sum(w.lens)}")
    m = measure_decode(w, steps, warmup, settle)
    nbytes = kv_bytes(w.lens, c["Hkv"], packed_bytes(c["D"], c["bwk"]), packed_bytes(c["D"], c["bwv"]))
    gbps = nbytes / (m["kernel_ms"] * 1e-3) / 1e9
    line = {"workload": f"BASELINE config {cfg}", "batch": len(w.lens), "q_heads": c["Hq"], "kv_heads": c["Hkv"],
            "seq_len": c["L"] or "U[512,65536]", "sum_seq_len": sum(w.lens), "bits_k": c["bwk"], "bits_v": c["bwv"],
            "table": c["table"], "data": workloads.DATA[c["data"]],
            "tokens_per_s": len(w.lens) / (m["ms_per_step"] * 1e-3), "us_per_step": m["ms_per_step"] * 1e3,
            "scan_kernel": scan_kernel_name(c), "scan_us": m["kernel_ms"] * 1e3, "algorithmic_bytes": nbytes,
            "scan_GBps": gbps, "frac": gbps / HBM_PEAK_GBPS,
            "step_frac": nbytes / (m["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, "splits": m["splits"],
            "pages_per_split": m["pages_per_split"], "steps": steps}
    if lds_rate:
        fl = lds_floor(w.lens, c, lds_rate, torch.cuda.get_device_properties(dev).multi_processor_count)
        line["lds_floor_us"] = fl["floor_us"]
        line["scan_over_lds_floor"] = line["scan_us"] / fl["floor_us"]
    if check:
        line["parity"] = parity(w)
    if tf32:
        line["allow_tf32"] = tf32_leg(w, nbytes, steps, warmup, settle, None, check)
    if prefill and c["bwk"] in (4, 6) and c["bwv"] in (4, 6):
        line["prefill"] = [prefill_bench(w, 16, check=check)]
    log(f"config {cfg}: {line}")
    del w
    torch.cuda.empty_cache()
    return line


def cpu_baseline(c, lens, q, kv, budget_s: float):
    """Oracle tiled CPU decode over a sample of page-table columns, scaled to the full step."""
    import torch
    from oracle import attention as oa

    # the host share this process may use (OMP_NUM_THREADS on the GPU box), not the whole machine
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(cores)
    cores = torch.get_num_threads()
    D, S, B = c["D"], c["S"], len(lens)
    width = kv.page_table_host.shape[1]

    def sample_kv(cols):
        ids = kv.page_table_host[:, :cols].reshape(-1).long()
        ids = ids.clamp(min=0)
        dev_ids = ids.to(kv.k_pages.device)
        table = torch.arange(B * cols, dtype=torch.int32).reshape(B, cols)
        s_lens = torch.tensor([min(L, cols * S) for L in lens], dtype=torch.int32)
        return oa.OracleKV(kv.k_pages[dev_ids].cpu(), kv.k_norms[dev_ids].cpu(), kv.v_pages[dev_ids].cpu(),
                           kv.v_norms[dev_ids].cpu(), table, s_lens,
                           oa.OracleQuant(kv.k_quant.Pi.cpu(), kv.k_quant.centroids.cpu(), kv.k_quant.bit_width),
                           oa.OracleQuant(kv.v_quant.Pi.cpu(), kv.v_quant.centroids.cpu(), kv.v_quant.bit_width),
                           D)

    qc = q.float().cpu()
    scale = oa.default_scale(D)
    # grow the sample until it holds about budget_s of CPU work (or the whole table)
    cols, dt = 4, 0.0
    while True:
        skv = sample_kv(cols)
        t0 = time.perf_counter()
        oa.tiled_compressed_attention(qc, skv, scale)
        dt = time.perf_counter() - t0
        if dt >= 0.5 * budget_s or cols >= width:
            break
        cols = int(min(width, max(2 * cols, cols * budget_s / max(dt, 1e-3))))
    t_step = dt / cols * width
    return {"value": B / t_step, "unit": "tokens/s", "cores": cores, "cpu_model": cpu_model(), "kind": "port",
            "sample": f"tiled_compressed_attention (torch CPU fp32) over {cols} of {width} page-table "
                      f"columns of the same batch ({dt:.1f} s), scaled x{width / cols:.1f} to the full step",
            "ms_per_step": t_step * 1e3}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--configs", default="3,4,5",
                    help="other BASELINE configs to measure in the same run (comma list, or 'none'): "
                         "scan time, roofline fraction, tokens/s and sampled parity per config")
    ap.add_argument("--config-steps", type=int, default=30, help="timed steps per extra config")
    ap.add_argument("--copies", type=int, default=2)
    ap.add_argument("--splits", type=int, default=None)
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work")
    ap.add_argument("--parity", choices=["on", "off"], default="on")
    ap.add_argument("--copy-peak", choices=["on", "off"], default="on")
    ap.add_argument("--dequant", choices=["on", "off"], default="on",
                    help="time the fused history dequantization at the reference's published shape "
                         "(N = 1,048,576 vectors, 4- and 6-bit)")
    ap.add_argument("--dequant-only", action="store_true",
                    help="run only the dequantization timing and print its JSON (for profiling that kernel)")
    ap.add_argument("--dense", choices=["on", "off"], default="on",
                    help="time the matched unquantized paged decode (bf16 pages) on the same shape")
    ap.add_argument("--append", choices=["on", "off"], default="on",
                    help="time the quantize+pack append of 16 new tokens per sequence (BASELINE config 3)")
    ap.add_argument("--traffic", choices=["on", "off"], default="on",
                    help="measure HBM bytes per scan launch with two rocprofv3 --pmc child runs")
    ap.add_argument("--tf32", choices=["on", "off"], default="on",
                    help="also time the reference's allow_tf32=True decode on the same pages (scan, "
                         "fraction of 8 TB/s, tokens/s, sampled parity), beside the default fp32-exact line")
    ap.add_argument("--prefill", choices=["on", "off"], default="on",
                    help="time the fused prefill over the packed pages (16 new tokens per sequence; "
                         "512 for the first two sequences) against the reference's dequantize + SDPA "
                         "route on the same pages, with its HBM and MFMA roofline and sampled parity")
    ap.add_argument("--lds-floor", choices=["on", "off"], default="on",
                    help="measure the LDS lookup rate (wn_probe_lds_lookup_rate, 8 waves per CU as the "
                         "row scans run) and report each scan's LDS floor beside its HBM roofline")
    ap.add_argument("--settle", type=float, default=0.5,
                    help="seconds of untimed steps before the warm-up, to reach sustained clocks")
    args = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); the "
              f"decode path has no collective: it would shard on the kv-head axis, one GPU's share "
              f"being this measurement", file=sys.stderr)
        return 2

    import torch
    from winnow_amd.packing import packed_bytes

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.dequant_only:
        deq = {**dequant_bench(dev), **dequant_bench(dev, fast=True)}
        cp = copy_peak(dev) if args.copy_peak == "on" else None
        print(json.dumps({"workload": "tq_dequant", "N": 1 << 20, "head_dim": 128, "out": "bf16", "results": deq,
                          "copy_peak": cp}))
        return 0
    t0 = time.time()
    w = workloads.build(args.config, dev, copies=args.copies, full_check=args.parity == "on")
    c, lens, q = w.c, w.lens, w.q
    log(f"workload config {args.config} built in {time.time() - t0:.1f} s: B={len(lens)} sum(L)={sum(lens)}")
    D, Hkv, Hq = c["D"], c["Hkv"], c["Hq"]
    bytes_step = kv_bytes(lens, Hkv, packed_bytes(D, c["bwk"]), packed_bytes(D, c["bwv"]))
    B = len(lens)
    m = measure_decode(w, args.steps, args.warmup, args.settle, args.splits)
    ms, kern_ms, ns, pps = m["ms_per_step"], m["kernel_ms"], m["splits"], m["pages_per_split"]
    log(f"step {ms * 1e3:.1f} us; page-scan kernel mean {kern_ms * 1e3:.1f} us "
        f"(median {m['kernel_ms_median'] * 1e3:.1f}); plan {ns} splits x {pps} pages")
    achieved = bytes_step / (kern_ms * 1e-3) / 1e9
    cp = copy_peak(dev) if args.copy_peak == "on" else None
    if cp:
        log(f"copy peak: {cp}")

    dense = None
    if args.dense == "on":
        dense = dense_bench(c, lens, q, dev)
        dense["packed_speedup_per_step"] = dense["us_per_step"] / (ms * 1e3)
        dense["packed_speedup_scan"] = dense["scan_kernel_us"] / (kern_ms * 1e3)
        log(f"dense: {dense}")
    app = append_bench(c, lens, w.table, w.quants, dev) if args.append == "on" else None
    if app:
        log(f"append: {app}")
    deq = {**dequant_bench(dev), **dequant_bench(dev, fast=True)} if args.dequant == "on" else None
    par = parity(w) if args.parity == "on" else None
    if par:
        log(f"parity: {par}")
    tf = None
    if args.tf32 == "on":
        # the reference's allow_tf32=True on the same pages: the TF32-class scan where it
        # is compiled (4 and 6-bit K and V on the row scan), else the same scan
        tf = tf32_leg(w, bytes_step, args.config_steps, min(args.warmup, 10), args.settle, args.splits,
                      args.parity == "on")
        log(f"allow_tf32: {tf}")
    pre = None
    if args.prefill == "on":
        pre = [prefill_bench(w, 16, check=args.parity == "on"),
               prefill_bench(w, 512, nseq=2, check=args.parity == "on")]
        log(f"prefill: {pre}")
    cpu = cpu_baseline(c, lens, q, w.kvs[0], args.cpu_budget) if args.cpu_baseline == "on" else None
    if cpu:
        log(f"cpu baseline: {cpu}")
    del w
    torch.cuda.empty_cache()
    traffic = hbm_traffic(args.config, scan_kernel_name(c)) if args.traffic == "on" else None
    if traffic:
        log(f"traffic: {traffic}")
    if tf and args.traffic == "on" and tf["kernel"] == "decode_rows_tf_kernel":
        tt = hbm_traffic(args.config, tf["kernel"], tf32=True)
        tf["traffic"] = tt["bytes_per_launch"] if tt else None
        tf["traffic_read_bytes"] = tt["FETCH_SIZE"]["bytes_per_launch"] if tt else None
        log(f"allow_tf32 traffic: {tt}")
    rate = lds_lookup_rate() if args.lds_floor == "on" else None
    ldsf = None
    if rate:
        ldsf = lds_floor(lens, c, rate, torch.cuda.get_device_properties(dev).multi_processor_count)
        ldsf["scan_over_floor"] = kern_ms * 1e3 / ldsf["floor_us"]
        log(f"lds floor: {ldsf}")
    others = {}
    extra = [] if args.configs in ("", "none") else [int(x) for x in args.configs.split(",")]
    for cfg in extra:
        if cfg != args.config:
            others[str(cfg)] = config_line(cfg, dev, args.config_steps, min(args.warmup, 10), args.settle,
                                           args.copies, args.parity == "on", rate, args.tf32 == "on",
                                           args.prefill == "on")

    result = {
        "metric": METRIC,
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_with_scan_events": m["ms_per_step_with_scan_events"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": DATA_NOTE + "; " + workloads.DATA[c["data"]],
        "config": {"workload": f"BASELINE config {args.config}", "batch": B, "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": D, "seq_len": c["L"] or "U[512,65536]", "sum_seq_len": sum(lens),
                   "page_size": c["S"], "bits_k": c["bwk"], "bits_v": c["bwv"], "table": c["table"],
                   "splits": ns, "pages_per_split": pps, "pool_copies": args.copies},
        "step_GBps": bytes_step / (ms * 1e-3) / 1e9,
        "kv_tokens_per_s": sum(lens) / (ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     # the same bytes over the whole decode step (rotate + scan + merge), the
                     # time the reference's traffic model divides by (bench_packed_attention.py:91-110)
                     "step_achieved": bytes_step / (ms * 1e-3) / 1e9,
                     "step_frac": bytes_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                     "target_us_at_0.70": bytes_step / (0.70 * HBM_PEAK_GBPS * 1e9) * 1e6,
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "traffic_read_bytes": traffic["FETCH_SIZE"]["bytes_per_launch"] if traffic else None,
                     "traffic_write_bytes": traffic["WRITE_SIZE"]["bytes_per_launch"] if traffic else None,
                     "counter_scale": {k: traffic[k]["factor"] for k in ("FETCH_SIZE", "WRITE_SIZE")}
                     if traffic else None,
                     "kernel": scan_kernel_name(c), "kernel_us": kern_ms * 1e3,
                     "algorithmic_bytes": bytes_step,
                     "copy_peak_GBps": cp["GBps"] if cp else None,
                     "frac_of_copy_peak": achieved / cp["GBps"] if cp else None},
        "lds_floor": ldsf,
        "cpu_baseline": cpu,
        "configs": others,
        "dense_baseline": dense,
        "append": app,
        "dequant": deq,
        "parity": par,
        "allow_tf32": tf,
        "prefill": pre,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
