"""Benchmark of the MoE decode block on one MI355X.

Workload (the metric's configuration): the Qwen3-30B-A3B-shaped MoE block
(hidden 2048, 128 experts, top-8 renormalised, SwiGLU intermediate 768) with
Q4 experts (group 64, the reference store format) at decode batch B=8.
A step is one call of the block for one layer over the batch.  Steps rotate
over 16 distinct synthetic layers (5.1 GB of expert bytes) so that neither
the L2 nor the 256 MB Infinity Cache holds the working set; the store is
resident in HBM before timing starts.

Reported (one JSON line):
  value        tokens/s of the block at B=8 (B * steps / elapsed)
  roofline     the whole block (the target is defined on it): algorithmic
               bytes per call (routed experts' Q4 records, router table, x in,
               out) / the event-timed call; peak 8 TB/s.  Beside it, under
               dominant_kernel, the same ratio for the gate/up expert kernel
               (the largest): its routed gate+up records / its average
               duration, measured with HIP events on the stream the kernels
               run on.  traffic: HBM bytes per call from two rocprofv3
               counter runs of this workload that the script starts before it
               touches the GPU (traffic_counters: per-kernel KiB, calibration
               and the ratio to the algorithmic bytes)
  stages       average milliseconds of each kernel
  router_margins  per token and layer, (p8 - p9) / p8 of the router softmax
               (how far each selection is from a tie)
  sweep        the same measurement at B=1 and B=32 (Qwen3), the headline
               batch at Q4 groups of 32 (qwen3_B8_G32), OLMoE B=1/8 (a
               float32 router table, as those configurations state; Q4
               groups of 64 and, as _G32, of 32), the
               prefill-style Qwen3 block: 512 tokens with Zipf(1.1)-biased
               routing, whose large segments take the MFMA branch, and the
               full 48-layer Qwen3-30B-A3B decode step at B=8 (attention over
               2049 cached positions + the MoE block per layer), with the MoE
               share of the step isolated; act_digits_5: the Qwen3 block at
               the headline B and at B=1 with 5 activation digit planes
               (the precise setting) instead of 4
  per_call_us  median, p10 and p90 of the per-call times (events between
               consecutive calls), for the headline and each sweep config
  parity       for the headline and every MoE config of the sweep, the timed
               workload against the oracle (oracle/): block outputs of every
               rotated layer (the Zipf block: layer 0), normwise per token
               max|gpu - oracle| / max|oracle| (the 1e-3 bar) and the
               elementwise p99 of |gpu - oracle| / |oracle| over outputs with
               |oracle| >= 1e-3 of the token's largest; router indices and
               weights compared bit for bit on every layer.  A config over the
               bar or with a routing mismatch makes the run exit non-zero.
  cpu_baseline the C restatement of the reference block (oracle/) in its
               AVX2 form (bit-identical to the scalar statement) on this
               host's cores as the reference runs it (inline at B=1, 8 pool
               workers + the caller above; batches in chunks of 16 tokens),
               on a bounded sample of the same workload: B=8 as the value,
               and under sweep Qwen3 B=1 (beside the reference's published
               1.19 ms), B=32, the Zipf 512-token batch and OLMoE B=1/8;
               sockets and the cores visible are reported
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
PEAK_MFMA_I8_TOPS = 5000.0     # dense int8 MFMA (the dense branch's operands)
ZIPF_ALPHA = 0.28              # Zipf(1.1) bias strength: per-expert counts about 5..200 over 512 tokens

# HBM traffic of the block's kernels: two rocprofv3 --pmc runs of this
# script on the default workload (FETCH_SIZE, then WRITE_SIZE; KiB per
# dispatch, averaged over every dispatch of each kernel), started before this
# process touches the GPU (measure_traffic).  Each counter is scaled by what
# it reads for a 256 MiB copy in the same run (FETCH_SIZE counts half of the
# copied bytes, WRITE_SIZE all of them on MI355X).
TRAFFIC_KERNELS = ("k_router_grp", "k_topk", "k_gateup", "k_down_comb")
TRAFFIC_ARGS = ["--no-sweep", "--cpu-seconds", "0", "--steps", "48", "--warmup", "16", "--calib-copy-mib", "256",
                "--no-traffic", "--no-parity"]
PARITY_TOL = 1e-3


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measure_traffic(batch: int, group: int, layers: int) -> dict:
    """HBM bytes per launch of the block's kernels, from two rocprofv3 --pmc
    runs of this script (one counter each) on the same workload with
    --calib-copy-mib 256.  Runs before this process initialises the GPU;
    returns the per-kernel KiB, the calibration factors and the scaled bytes,
    or the reason it could not."""
    import csv
    import shutil
    import subprocess
    import tempfile
    from collections import defaultdict

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return {"error": "rocprofv3 not found"}
    tmp = tempfile.gettempdir()
    tail = [sys.executable, str(ROOT / "bench.py"), *TRAFFIC_ARGS, "--batch", str(batch), "--group", str(group),
            "--layers", str(layers)]
    kib, factor = {}, {}
    calib_kib = 256 * 1024.0
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="jm_pmc_", dir=tmp)
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--", *tail]
        log(f"traffic: {counter} run ({' '.join(cmd[:4])} ... -- bench.py {' '.join(TRAFFIC_ARGS[:6])} ...)")
        try:
            r = subprocess.run(cmd, cwd=tmp, env={**os.environ, "TMPDIR": tmp}, stdout=subprocess.DEVNULL,
                               stderr=subprocess.PIPE, timeout=240)
            rc = r.returncode
        except subprocess.TimeoutExpired:
            shutil.rmtree(d, ignore_errors=True)
            return {"error": f"{counter} run timed out"}
        files = sorted(Path(d).rglob("*counter_collection.csv"))
        if not files:
            shutil.rmtree(d, ignore_errors=True)
            return {"error": f"{counter} run wrote no counter file (exit {rc})"}
        vals = defaultdict(list)
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                vals[row["Kernel_Name"]].append(float(row["Counter_Value"]))
        shutil.rmtree(d, ignore_errors=True)
        per = {}
        for k in TRAFFIC_KERNELS:
            v = [x for name, xs in vals.items() if k + "<" in name or name.endswith(k) for x in xs]
            per[k] = sum(v) / len(v) if v else None
        cp = [x for name, xs in vals.items() if "copyBuffer" in name for x in xs if x > 0.25 * calib_kib]
        if not cp or any(per[k] is None for k in TRAFFIC_KERNELS):
            return {"error": f"{counter}: kernels or the calibration copy missing from the counter file"}
        kib[counter] = per
        factor[counter] = calib_kib / (sum(cp) / len(cp))
        log(f"traffic: {counter} KiB per dispatch {per}, calibration factor {factor[counter]:.3f} (exit {rc})")
    scaled = {k: 1024.0 * (kib["FETCH_SIZE"][k] * factor["FETCH_SIZE"] + kib["WRITE_SIZE"][k] * factor["WRITE_SIZE"])
              for k in TRAFFIC_KERNELS}
    return {"fetch_kib": kib["FETCH_SIZE"], "write_kib": kib["WRITE_SIZE"],
            "fetch_factor": factor["FETCH_SIZE"], "write_factor": factor["WRITE_SIZE"],
            "bytes": scaled, "block_bytes": sum(scaled.values()),
            "command": f"rocprofv3 --pmc <FETCH_SIZE|WRITE_SIZE> --output-format csv -d <dir> -o run -- "
                       f"python3 bench.py {' '.join(TRAFFIC_ARGS)} --batch {batch} --group {group} --layers {layers}"}


def percentiles_us(times_ms) -> dict:
    import numpy as np

    t = np.asarray(times_ms, dtype=np.float64) * 1e3
    return {"median": float(np.median(t)), "p10": float(np.percentile(t, 10)), "p90": float(np.percentile(t, 90)),
            "calls": int(t.size)}


def normwise(out, ref) -> float:
    """max over tokens of max_i |out - ref| / max_i |ref| (the 1e-3 bar)."""
    import numpy as np

    den = np.abs(ref).max(axis=1)
    num = np.abs(out.astype(np.float64) - ref.astype(np.float64)).max(axis=1)
    return float(np.max(num / np.where(den > 0, den, 1.0)))


def elementwise_p99(out, ref) -> float:
    """p99 of |out - ref| / |ref| over the outputs with |ref| >= 1e-3 of the
    token's largest."""
    import numpy as np

    big = np.abs(ref) >= 1e-3 * np.abs(ref).max(axis=1, keepdims=True)
    rel = np.abs(out.astype(np.float64) - ref)[big] / np.abs(ref)[big]
    return float(np.percentile(rel, 99)) if rel.size else 0.0


def block_parity(store, moes, x_np, layers) -> dict:
    """The timed workload against the oracle: block outputs, router indices
    and weights of each layer in `layers` for the tokens x_np."""
    import numpy as np
    import torch

    from oracle import oracle as O

    B, k = x_np.shape[0], store.shape.topk
    x = torch.from_numpy(x_np).cuda()
    out = torch.empty_like(x)
    top = torch.empty((B, k), dtype=torch.int32, device="cuda")
    tw = torch.empty((B, k), dtype=torch.float32, device="cuda")
    threads = min(9, max(1, O.cpu_count()))
    nerr, p99, top_ok, tw_ok = 0.0, 0.0, 0, 0
    for l in layers:
        store.layer_ffn_batch(l, x, out, topk_idx=top, topk_w=tw)
        o, t, w = out.cpu().numpy(), top.cpu().numpy(), tw.cpu().numpy()
        ro, rt, rw = moes[l].forward(x_np, n_threads=threads)
        top_ok += int(np.array_equal(t, rt))
        tw_ok += int(np.array_equal(w.view(np.uint32), rw.view(np.uint32)))
        nerr = max(nerr, normwise(o, ro))
        p99 = max(p99, elementwise_p99(o, ro))
    n = len(layers)
    return {"layers_checked": n, "normwise_max": nerr, "elementwise_p99_max": p99,
            "topk_bitexact_layers": top_ok, "weights_bitexact_layers": tw_ok,
            "ok": bool(nerr <= PARITY_TOL and top_ok == n and tw_ok == n)}


def build_layers(shape, n_layers, group, seed, router_bf16=True):
    import numpy as np
    import torch

    from joule_amd.moe import HbmExpertStore
    from joule_amd.synth import router_weights, torch_store

    blob, offsets = torch_store(shape, n_layers, group, seed)
    store = HbmExpertStore(shape, n_layers, blob, offsets, group)
    gw = np.stack([router_weights(shape, l, bf16=router_bf16) for l in range(n_layers)])
    store.set_router(torch.from_numpy(gw).cuda())
    torch.cuda.synchronize()
    return store, gw


def routed_experts(store, n_layers, x):
    """Distinct experts each layer routes this batch to (counted from a run)."""
    import numpy as np
    import torch

    B = x.shape[0]
    k = store.shape.topk
    top = torch.empty((B, k), dtype=torch.int32, device="cuda")
    U = []
    for l in range(n_layers):
        store.layer_ffn_batch(l, x, topk_idx=top)
        t = top.cpu().numpy()
        U.append(len(np.unique(t[t >= 0])))
    return U


def measure(store, gw, x, steps, warmup, n_layers, stage_steps=None):
    """(ms_per_step, per-stage ms averages, routed experts per layer,
    per-call time percentiles)."""
    import torch

    from joule_amd._lib import STAGES

    out = torch.empty_like(x)
    store.reserve(x.shape[0])
    for i in range(warmup):
        store.layer_ffn_batch(i % n_layers, x, out)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        store.layer_ffn_batch(i % n_layers, x, out)
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the per-call distribution: the same calls with an event between each two
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record(st)
    for i in range(steps):
        store.layer_ffn_batch(i % n_layers, x, out)
        evs[i + 1].record(st)
    torch.cuda.synchronize()
    dist = percentiles_us([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)])
    # per-kernel durations: same calls with an event before/after each kernel
    store.profile(True)
    acc = {k: 0.0 for k in STAGES}
    ns = stage_steps or steps
    for i in range(ns):
        store.layer_ffn_batch(i % n_layers, x, out)
        for k, v in store.stage_ms().items():
            acc[k] += v
    store.profile(False)
    stages = {k: v / ns for k, v in acc.items()}
    U = routed_experts(store, n_layers, x)
    return ms, stages, U, dist


def block_numbers(shape, group, B, ms, stages, U, steps, n_layers, router_bytes=4):
    from joule_amd.moe import algorithmic_bytes
    from joule_amd.q4_store import record_sizes

    # average routed experts over the timed steps' layer sequence
    seq = [U[i % n_layers] for i in range(steps)]
    u_avg = sum(seq) / len(seq)
    bytes_block = algorithmic_bytes(shape, group, B, 0, router_bytes) + u_avg * sum(
        sum(record_sizes(r, c, group)) for r, c in ((shape.m, shape.d), (shape.m, shape.d), (shape.d, shape.m)))
    gate_up = u_avg * 2 * sum(record_sizes(shape.m, shape.d, group))
    down = u_avg * sum(record_sizes(shape.d, shape.m, group))
    return {
        "B": B,
        "tok_per_s": B / (ms * 1e-3),
        "ms_per_step": ms,
        "experts_routed_avg": u_avg,
        "bytes_alg": bytes_block,
        "block_GBs": bytes_block / (ms * 1e-3) / 1e9,
        "block_frac": bytes_block / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "gateup_bytes": gate_up,
        "gateup_GBs": gate_up / (stages["gateup"] * 1e-3) / 1e9,
        "down_bytes": down,
        "down_GBs": down / (stages["down"] * 1e-3) / 1e9,
        "stages_ms": stages,
    }


def zipf_block(store, gw, steps, n_layers, bz=512, check=True):
    """The prefill-style Qwen3 block: bz tokens with Zipf(1.1)-biased routing
    (per-expert counts about 5..200 at bz = 512); the experts with at least
    dense_min (8) slots take the MFMA branch.  With check, layer 0's block
    is compared with the oracle.  Returns (results, biased router table,
    biased x)."""
    import numpy as np
    import torch

    from joule_amd.synth import activations, apply_logit_bias, zipf_bias

    shape, G = store.shape, store.group
    rb = store.router_bytes_per_weight()
    bias = zipf_bias(shape.E, s=1.1, alpha=ZIPF_ALPHA)
    xz_np = activations(bz, shape.d)
    gz = np.stack([apply_logit_bias(gw[l], xz_np, bias)[0] for l in range(n_layers)])
    xz_np = apply_logit_bias(gw[0], xz_np, bias)[1]
    xz = torch.from_numpy(xz_np).cuda()
    store.set_router(torch.from_numpy(gz).cuda())
    nz = max(steps // 2, 100)
    m2, st2, U2, dist = measure(store, gz, xz, nz, 10, n_layers, stage_steps=min(nz, 50))
    r = block_numbers(shape, G, bz, m2, st2, U2, nz, n_layers, rb)
    top = torch.empty((bz, shape.topk), dtype=torch.int32, device="cuda")
    store.layer_ffn_batch(0, xz, topk_idx=top)
    tiles = store.dense_tiles()
    counts = np.bincount(top.cpu().numpy().ravel(), minlength=shape.E)
    flops = 2.0 * bz * shape.topk * 3 * shape.d * shape.m
    res = {
        **{k: r[k] for k in ("tok_per_s", "ms_per_step", "block_GBs", "block_frac", "experts_routed_avg")},
        "tflops": flops / (m2 * 1e-3) / 1e12,
        "mfma_frac_of_int8_peak": flops / (m2 * 1e-3) / 1e12 / PEAK_MFMA_I8_TOPS,
        "zipf_alpha": ZIPF_ALPHA, "count_max": int(counts.max()), "count_min": int(counts.min()),
        "dense_experts": int((counts >= 8).sum()), "dense_tiles": tiles,
        "stages_ms": st2, "per_call_us": dist,
    }
    if check:
        res["parity"] = block_parity(store, oracle_moes(store, gz, 1), xz_np, [0])
        log(f"parity qwen3 zipf B={bz}: {res['parity']}")
    log(f"sweep qwen3 zipf B={bz}: {r['tok_per_s']:.0f} tok/s, {m2 * 1e3:.1f} us/step, "
        f"{flops / (m2 * 1e-3) / 1e12:.1f} TFLOP/s, counts {counts.min()}..{counts.max()}, "
        f"dense tiles {tiles}, stages {st2}")
    store.set_router(torch.from_numpy(gw).cuda())
    return res, gz, xz_np


def host_info() -> dict:
    """CPU model, sockets and the cores this process may run on."""
    import os as _os

    model, phys = "unknown", set()
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name") and model == "unknown":
                model = ln.split(":", 1)[1].strip()
            elif ln.startswith("physical id"):
                phys.add(ln.split(":", 1)[1].strip())
    except OSError:
        pass
    cores = sorted(_os.sched_getaffinity(0))
    runs, start = [], None
    for i, c in enumerate(cores):
        if start is None:
            start = c
        if i + 1 == len(cores) or cores[i + 1] != c + 1:
            runs.append(f"{start}-{c}" if c != start else f"{c}")
            start = None
    return {"model": model, "sockets": len(phys) or 1, "cpus_visible": len(cores),
            "affinity": ",".join(runs),
            "pinning": "threads not pinned (the reference starts 8 pool workers with no affinity, decoder3.py:135, decode_kernel.c:631-656)"}


def cpu_time(moes, x_np, threads, budget_s, min_calls=3, chunk=16):
    """Median seconds of one block call of the oracle (the C restatement of
    layer_ffn_batch) over B = x_np.shape[0] tokens, run as the reference
    runs a batch: chunks of at most 16 tokens (decode_layers_batch clamps B
    to BMAX = 16, decode_kernel.c:1522), rotating layers.  Returns (median,
    calls, top-k of the first call)."""
    import numpy as np

    B = x_np.shape[0]
    chunks = [x_np[i:i + chunk] for i in range(0, B, chunk)]
    first = [moes[0].forward(c, n_threads=threads, all_tokens=True)[1] for c in chunks]   # warm-up, pool start
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while (time.perf_counter() < t_end and i < 400) or i < min_calls:
        t0 = time.perf_counter()
        for c in chunks:
            moes[i % len(moes)].forward(c, n_threads=threads, all_tokens=True)
        times.append(time.perf_counter() - t0)
        i += 1
    return float(np.median(times)), len(times), np.concatenate(first)


def oracle_moes(store, gw, n_layers):
    from oracle import oracle as O

    s = store.shape
    host = store.blob.cpu().numpy()
    return [O.OracleMoE(s.d, s.m, s.E, s.topk, s.renorm, store.group, gw[l], host,
                        store.offsets[:, l * s.E:(l + 1) * s.E]) for l in range(n_layers)]


def cpu_case(moes, x_np, budget_s, label, min_calls=3):
    """One CPU baseline figure at the reference's thread count for the batch:
    inline at B = 1 (decode_kernel.c:1496-1497), otherwise the decoder's 8
    pool workers + the caller (decoder3.py:135, decode_kernel.c:1499)."""
    from joule_amd.moe import QWEN3
    from oracle import oracle as O

    B = x_np.shape[0]
    threads = min(9 if B > 1 else 1, max(1, O.cpu_count()))
    # the AVX2 form of the row and router dots (the reference's B <= 16
    # path is AVX2, decode_kernel.c:774-822), bit-identical to the scalar
    # statement of the same per-lane order
    O.set_simd(True)
    med, n, top = cpu_time(moes, x_np, threads, budget_s, min_calls)
    log(f"CPU baseline {label}: {B / med:.1f} tok/s, {med * 1e3:.2f} ms per block call on {threads} threads")
    r = {"value": B / med, "unit": "tokens/s", "cores": threads, "ms_per_call": med * 1e3, "calls": n,
         "chunks_of_16": (B + 15) // 16, "form": "avx2"}
    if B == 1 and moes[0].d == QWEN3.d and moes[0].E == QWEN3.E:
        # the reference's published B=1 block: AVX2, one thread, on a
        # Ryzen AI 7 350 (results/VALIDATION_LOG.md:1352-1356)
        r["reference_published_ms_per_call"] = 1.19
        r["vs_reference_published"] = med * 1e3 / 1.19
    return r, top


def cpu_baseline(moes, x_np, budget_s, gpu_top):
    """The oracle on the host cores for the metric's batch (B = 8, 8 workers
    + caller as the reference runs B > 1), for about budget_s seconds.  The
    oracle's top-k of the first layer is compared with the GPU's."""
    import numpy as np

    r, top = cpu_case(moes, x_np, budget_s, f"qwen3 B={x_np.shape[0]}")
    h = host_info()
    r.update({
        "kind": "port",
        "sample": (f"{r['calls']} calls of the Qwen3-shaped block at B={x_np.shape[0]} rotating {len(moes)} "
                   f"layers, median {r['ms_per_call']:.2f} ms/call; AVX2 form of the restatement, every token "
                   f"dotted on every routed expert row as the reference kernel does; host {h['model']}, "
                   f"{h['sockets']} socket(s), "
                   f"{h['cpus_visible']} cpus visible ({h['affinity']}), threads unpinned"),
        "host": h,
        "topk_bitexact_vs_gpu": bool(np.array_equal(top, gpu_top)),
    })
    return r


def router_margins(store, n_layers, x):
    """Per layer and token: (p_k - p_(k+1)) / p_k of the router softmax, the
    gap between the last selected expert's probability and the first
    unselected one's (decode_kernel.c:1433-1441 selects by strict >, so a
    gap near zero is where a rounding-level change of a logit could change
    the selection).  Read from the GPU's logits."""
    import numpy as np
    import torch

    from joule_amd import _lib

    B, k, E = x.shape[0], store.shape.topk, store.shape.E
    lg = torch.empty((B, E), dtype=torch.float32, device="cuda")
    res = []
    for l in range(n_layers):
        store.layer_ffn_batch(l, x)
        _lib.check(_lib.lib().jm_store_copy_workspace(store._h, _lib.WS_LOGITS, _lib.ptr(lg), lg.numel() * 4,
                                                      _lib.stream_handle()), "jm_store_copy_workspace")
        z = lg.cpu().numpy().astype(np.float64)
        p = np.exp(z - z.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        q = -np.sort(-p, axis=1)
        res.append((q[:, k - 1] - q[:, k]) / q[:, k - 1])
    m = np.array(res)
    return {"definition": "(p_k - p_k+1) / p_k per token, k = 8, from the GPU router logits",
            "min": float(m.min()), "below_1e-4": int((m < 1e-4).sum()), "count": int(m.size),
            "per_layer_token": [[float(f"{v:.4g}") for v in row] for row in m]}


def decode_step(B, steps, warmup, group, n_layers=48, position=2048, maxT=2176, kv_f32=False):
    """The full Qwen3-30B-A3B-shaped decode step: n_layers x (attention + MoE
    block) at batch B, every token at cache position `position` (attention
    over position + 1 rows of a bf16 cache, or with kv_f32 a float32 one,
    filled with N(0, 1)).  Returns tokens/s, the attention / MoE split of a
    profiled step, and the algorithmic HBM bytes of a step (routed experts
    counted per layer)."""
    import numpy as np
    import torch

    from joule_amd.decoder import DecoderWeights, HipDecoder, KVCacheSet, qwen3_30b_a3b
    from joule_amd.moe import QWEN3
    from joule_amd.q4_store import record_sizes
    from joule_amd.synth import activations, decoder_weights, fill_kv

    shape = qwen3_30b_a3b(n_layers, maxT)
    log(f"decode: building {n_layers} Qwen3-30B-A3B layers (store, attention weights, KV cache)")
    store, _ = build_layers(QWEN3, n_layers, group, seed=1000)
    weights = DecoderWeights(shape, **decoder_weights(shape))
    kv_dtype = torch.float32 if kv_f32 else torch.bfloat16
    kv = KVCacheSet(shape, B, dtype=kv_dtype)
    fill_kv(kv.data)
    dec = HipDecoder(store, weights)
    x = torch.from_numpy(activations(B, shape.d)).cuda()
    hid = torch.empty_like(x)
    pos = [position] * B
    store.reserve(B)
    for _ in range(warmup):
        dec.decode_layers_batch(x, pos, kv, hid)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(steps):
        dec.decode_layers_batch(x, pos, kv, hid)
    e1.record(st)
    host_ms = (time.perf_counter() - t0) * 1e3 / steps      # enqueue time per step
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record(st)
    for i in range(steps):
        dec.decode_layers_batch(x, pos, kv, hid)
        evs[i + 1].record(st)
    torch.cuda.synchronize()
    dist = percentiles_us([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)])
    # attention / MoE split (events at every layer's boundaries)
    store.profile(True)
    split = {"attention": 0.0, "moe": 0.0, "total": 0.0}
    for _ in range(3):
        dec.decode_layers_batch(x, pos, kv, hid)
        for k, v in dec.split_ms().items():
            split[k] += v / 3
    store.profile(False)
    # routed experts per layer, from a traced step
    k = QWEN3.topk
    tr = torch.empty((n_layers, B, k), dtype=torch.int32, device="cuda")
    dec.trace_topk(tr)
    dec.decode_layers_batch(x, pos, kv, hid)
    dec.trace_topk(None)
    t = tr.cpu().numpy()
    U = [len(np.unique(t[l])) for l in range(n_layers)]
    eb = sum(sum(record_sizes(r, c, group)) for r, c in ((QWEN3.m, QWEN3.d), (QWEN3.m, QWEN3.d), (QWEN3.d, QWEN3.m)))
    H, KH, hd, d = shape.n_heads, shape.n_kv, shape.hd, shape.d
    T = position + 1
    moe_bytes = sum(U) * eb + n_layers * (QWEN3.E * d * store.router_bytes_per_weight() + 2 * B * d * 4)
    attn_w = n_layers * 2 * (H * hd * d + 2 * KH * hd * d + d * H * hd)
    kv_bytes = n_layers * B * T * KH * hd * 2 * kv.data.element_size()
    total = moe_bytes + attn_w + kv_bytes
    ok = bool(torch.isfinite(hid).all().item())
    # the serve path: the same step ending in the lm_head (vocabulary 151936,
    # bf16 N(0, 0.02)) and its argmax, tokens out
    g = torch.Generator(device="cuda")
    g.manual_seed(7000)
    lm = (torch.randn((shape.V, shape.d), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    dec.set_lm_head(lm)
    del lm
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    for _ in range(warmup):
        dec.decode_layers_batch_argmax(x, pos, kv, tok)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(steps):
        dec.decode_layers_batch_argmax(x, pos, kv, tok)
    e1.record(st)
    torch.cuda.synchronize()
    ms_lm = e0.elapsed_time(e1) / steps
    # the lm_head + argmax alone, on the step's hidden state
    n_lm = 20
    e0.record(st)
    for _ in range(n_lm):
        dec.lm_head(hid, None, tok)
    e1.record(st)
    torch.cuda.synchronize()
    lm_ms = e0.elapsed_time(e1) / n_lm
    lm_bytes = shape.V * shape.d * 2
    # prefill: one 512-token prompt through every layer in one pass per
    # layer (jm_prefill_layers), against the reference's loop of one decode
    # step per position, estimated from B=1 decode steps on these kernels
    Tp = 512
    dec.weights.t["embed"] = (torch.randn((shape.V, shape.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    dec._w = dec.weights.kernel_w()
    prompt = torch.randint(0, shape.V, (Tp,), generator=g, device="cuda", dtype=torch.int32)
    kvp = KVCacheSet(shape, 1, dtype=kv_dtype)
    plog = torch.empty(shape.V, dtype=torch.float32, device="cuda")
    dec.prefill_layers(prompt, kvp, 0, plog)
    torch.cuda.synchronize()
    n_pf = 3
    e0.record(st)
    for _ in range(n_pf):
        dec.prefill_layers(prompt, kvp, 0, plog)
    e1.record(st)
    torch.cuda.synchronize()
    pf_ms = e0.elapsed_time(e1) / n_pf
    x1 = x[:1].contiguous()
    for _ in range(warmup):
        dec.decode_layers_batch(x1, [Tp - 1], kvp, hid[:1])
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(steps):
        dec.decode_layers_batch(x1, [Tp - 1], kvp, hid[:1])
    e1.record(st)
    torch.cuda.synchronize()
    b1_ms = e0.elapsed_time(e1) / steps
    del kvp
    res = {
        "tok_per_s": B / (ms * 1e-3), "ms_per_step": ms, "per_step_us": dist, "host_enqueue_ms_per_step": host_ms,
        "layers": n_layers, "batch": B, "position": position, "kv_cache": "f32" if kv_f32 else "bf16",
        "attention_ms_profiled": split["attention"], "moe_ms_profiled": split["moe"],
        "step_ms_profiled": split["total"],
        "moe_share": split["moe"] / split["total"] if split["total"] > 0 else None,
        "experts_routed_avg": sum(U) / len(U),
        "bytes_alg": total, "bytes_moe": moe_bytes, "bytes_attn_weights": attn_w, "bytes_kv": kv_bytes,
        "GBs": total / (ms * 1e-3) / 1e9, "hbm_frac": total / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "hidden_finite": ok,
        "prefill_512": {
            "prompt_tokens": Tp, "ms": pf_ms, "tok_per_s": Tp / (pf_ms * 1e-3),
            "decode_B1_ms_per_step": b1_ms,
            "per_position_loop_ms_estimate": Tp * b1_ms,
            "speedup_vs_per_position_loop": Tp * b1_ms / pf_ms,
        },
        "with_lm_head_argmax": {
            "tok_per_s": B / (ms_lm * 1e-3), "ms_per_step": ms_lm, "vocab": shape.V,
            "lm_head_argmax_ms": lm_ms, "lm_head_bytes": lm_bytes,
            "lm_head_GBs": lm_bytes / (lm_ms * 1e-3) / 1e9,
            "bytes_alg": total + lm_bytes,
            "GBs": (total + lm_bytes) / (ms_lm * 1e-3) / 1e9,
        },
    }
    log(f"decode {n_layers} layers B={B} ({res['kv_cache']} cache): {res['tok_per_s']:.0f} tok/s, {ms:.3f} ms/step "
        f"(host enqueue {host_ms:.3f} ms), attention {split['attention']:.3f} ms, MoE {split['moe']:.3f} ms, "
        f"{res['GBs']:.0f} GB/s over {total / 1e9:.2f} GB; with lm_head + argmax {B / (ms_lm * 1e-3):.0f} tok/s "
        f"({ms_lm:.3f} ms/step; lm_head {lm_ms * 1e3:.1f} us, {lm_bytes / (lm_ms * 1e-3) / 1e9:.0f} GB/s); "
        f"prefill {Tp} tokens {pf_ms:.1f} ms ({Tp / (pf_ms * 1e-3):.0f} tok/s) vs {Tp * b1_ms:.0f} ms "
        f"for {Tp} B=1 decode steps")
    store.close()
    del dec, weights, kv, store
    torch.cuda.empty_cache()
    return res


def monotone_stats(times):
    """(non-decreasing, the largest amount by which a time exceeds a later one)
    for times in the order of increasing size."""
    inv = max((times[i] - min(times[i + 1:]) for i in range(len(times) - 1)), default=0.0)
    return all(b >= a for a, b in zip(times, times[1:])), max(0.0, inv)


def plugin_q4_gemm(group, m=768, d=2048, sizes=(1, 2, 4, 6, 7, 8, 12, 16, 20, 24, 28, 32, 33, 36, 48, 64, 512),
                   reps=100, rounds=5):
    """The plugin product HipBackend.q4_gemm (jm_q4_gemm_f32, the reference's
    q4_gemm_f32) on one Qwen3 expert matrix shape (m=768 rows of d=2048),
    at each token count T (inputs and the packed matrix resident on the GPU;
    the workspace cached after the first call), with the library's own
    choice of kernel and with each of the two kernels forced (the v_dot8
    digit kernel, the int8 matrix cores), from which the crossover is read.

    `us_per_call` is the GPU's time per call: a bounded spin kernel
    (torch.cuda._sleep) holds the stream while the host enqueues the `reps`
    calls, so that they run back to back whatever the host's pace; an event
    query after the enqueue confirms that the GPU had not reached the calls
    yet (`queued_ahead`).  Median of `rounds` such runs.  `host_paced_us`
    is the same calls enqueued with the stream idle (each call's host work
    and launches on the critical path: the rate a caller issuing one call
    after another sees), and at T = 1 the host-side time of one call
    enqueued and waited for is reported too."""
    import numpy as np
    import torch

    from joule_amd import _lib
    from joule_amd import q4_store as q4
    from joule_amd.backend import HipBackend

    L = _lib.lib()
    rng = np.random.default_rng(7)
    sb, pb = q4.quantize(rng.normal(0, 0.02, (m, d)).astype(np.float32), group)
    sc = torch.from_numpy(np.frombuffer(sb, np.uint16).copy().view(np.int16)).cuda()
    pk = torch.from_numpy(np.frombuffer(pb, np.uint8).copy()).cuda()
    be = HipBackend()
    st = torch.cuda.current_stream()
    default_min = L.jm_get_q4_gemm_min_tokens()

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    # the spin kernel's microseconds per requested cycle
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    e0.record(st)
    torch.cuda._sleep(1_000_000)
    e1.record(st)
    torch.cuda.synchronize()
    us_per_cycle = e0.elapsed_time(e1) * 1e3 / 1_000_000

    def run(y, X, hold_cycles):
        if hold_cycles:
            torch.cuda._sleep(hold_cycles)
        e0.record(st)
        t0 = time.perf_counter()
        for _ in range(reps):
            be.q4_gemm(y, X, pk, sc, m, d, group)
        host_us = (time.perf_counter() - t0) * 1e6
        e1.record(st)
        ahead = not e0.query()          # the GPU still in the spin when the last call was enqueued
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps, host_us, ahead

    def time_calls(y, X, min_t):
        """(GPU us per call, its spread over the rounds, host-paced us per
        call, every run queued ahead)"""
        _lib.check(L.jm_set_q4_gemm_min_tokens(min_t), "jm_set_q4_gemm_min_tokens")
        for _ in range(5):
            be.q4_gemm(y, X, pk, sc, m, d, group)
        torch.cuda.synchronize()
        paced, host_us, _ = run(y, X, 0)
        # hold the stream for twice the host's enqueue time of the calls
        hold = max(1000, int(2.0 * host_us / us_per_cycle))
        gpu, ahead = [], True
        for _ in range(rounds):
            us, _, a = run(y, X, hold)
            gpu.append(us)
            ahead = ahead and a
        return float(np.median(gpu)), float(max(gpu) - min(gpu)), paced, ahead

    out = {}
    try:
        for T in sizes:
            X = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).cuda()
            y = torch.empty((T, m), dtype=torch.float32, device="cuda")
            dot8_us, _, _, a1 = time_calls(y, X, 1 << 30)
            mfma_us, _, _, a2 = time_calls(y, X, 1)
            us, spread, paced, a3 = time_calls(y, X, 0)
            nbytes = m * d // 2 + m * (d // group) * 2 + T * d * 4 + T * m * 4
            path = "mfma_i8" if T >= default_min else "dot8_digits"
            out[f"T{T}"] = {"us_per_call": us, "spread_us": spread, "host_paced_us": paced, "bytes": nbytes,
                            "GBs": nbytes / (us * 1e-6) / 1e9, "path": path,
                            "dot8_us": dot8_us, "mfma_us": mfma_us, "queued_ahead": a1 and a2 and a3,
                            "tflops_equiv": 2.0 * T * m * d / (us * 1e-6) / 1e12}
            log(f"plugin q4_gemm m={m} d={d} T={T}: {us:.2f} us ({path}; host-paced {paced:.2f}); "
                f"dot8 {dot8_us:.2f}, mfma {mfma_us:.2f}")
            if T == 1:
                # host-side: each call enqueued and waited for
                hs = []
                for _ in range(50):
                    t0 = time.perf_counter()
                    be.q4_gemm(y, X, pk, sc, m, d, group)
                    torch.cuda.synchronize()
                    hs.append((time.perf_counter() - t0) * 1e6)
                out["T1"]["host_us_per_call_synced"] = float(np.median(hs))
    finally:
        L.jm_set_q4_gemm_min_tokens(0)
    # the smallest T from which the matrix cores are no slower at every larger measured T
    ts = [int(k[1:]) for k in out]
    cross = None
    for t in ts:
        if all(out[f"T{u}"]["mfma_us"] <= out[f"T{u}"]["dot8_us"] for u in ts if u >= t):
            cross = t
            break
    monotone, inversion = monotone_stats([out[f"T{t}"]["us_per_call"] for t in ts])
    return {"m": m, "d": d, "group": group, "default_min_tokens": default_min, "measured_crossover_T": cross,
            "us_per_call_monotone_in_T": monotone,
            # the most by which a size's time exceeds that of a larger size (sizes within one
            # 32-token tile do the same work on the matrix cores and differ by noise)
            "max_inversion_us": inversion,
            "queued_ahead": all(v["queued_ahead"] for v in out.values()), "sizes": out}


def dense_step(B, steps, warmup, n_layers=36, position=2048, maxT=2176):
    """A dense model's decode step (layer_ffn_batch's E == 0 branch in every
    layer): Qwen3-8B-shaped layers (hidden 4096, GQA 32 / 8 heads of 128,
    per-head QK-norm, FFN intermediate 12288, bf16 weights N(0, 0.02)),
    every token at cache position `position` of a bf16 cache.  Returns
    tokens/s and the step's algorithmic bytes (weights once, KV rows)."""
    import torch

    from joule_amd.decoder import DecoderShape, DecoderWeights, HipDecoder, KVCacheSet
    from joule_amd.dense import DenseFfnStore, dense_ffn_shape
    from joule_amd.synth import activations, decoder_weights, fill_kv

    d, m, H, KH, hd = 4096, 12288, 32, 8, 128
    shape = DecoderShape(n_layers=n_layers, moe=dense_ffn_shape(d, m), n_heads=H, n_kv=KH, maxT=maxT,
                         qk_norm_type=1, name="qwen3-8b-shaped")
    log(f"dense decode: building {n_layers} Qwen3-8B-shaped layers")
    store = DenseFfnStore(d, m, n_layers)
    dec = HipDecoder(store, DecoderWeights(shape, **decoder_weights(shape)))
    kv = KVCacheSet(shape, B)
    fill_kv(kv.data)
    x = torch.from_numpy(activations(B, d)).cuda()
    hid = torch.empty_like(x)
    pos = [position] * B
    for _ in range(warmup):
        dec.decode_layers_batch(x, pos, kv, hid)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        dec.decode_layers_batch(x, pos, kv, hid)
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    w_bytes = n_layers * 2 * (H * hd * d + 2 * KH * hd * d + d * H * hd + 3 * m * d)
    kv_bytes = n_layers * B * (position + 1) * KH * hd * 2 * 2
    total = w_bytes + kv_bytes
    ok = bool(torch.isfinite(hid).all().item())
    res = {"tok_per_s": B / (ms * 1e-3), "ms_per_step": ms, "layers": n_layers, "batch": B, "position": position,
           "bytes_alg": total, "GBs": total / (ms * 1e-3) / 1e9,
           "hbm_frac": total / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "hidden_finite": ok}
    log(f"dense decode {n_layers} layers B={B}: {res['tok_per_s']:.0f} tok/s, {ms:.3f} ms/step, "
        f"{res['GBs']:.0f} GB/s over {total / 1e9:.2f} GB")
    del dec, kv, store
    torch.cuda.empty_cache()
    return res


def prefill_only(group, reps, n_layers=48, maxT=2176, Tp=512):
    """Only the 512-token prefill of decode_step's model (for kernel
    profiles): one warm-up pass, then `reps` timed passes of
    jm_prefill_layers with the lm_head at the last position."""
    import torch

    from joule_amd.decoder import DecoderWeights, HipDecoder, KVCacheSet, qwen3_30b_a3b
    from joule_amd.moe import QWEN3
    from joule_amd.synth import decoder_weights

    shape = qwen3_30b_a3b(n_layers, maxT)
    log(f"prefill: building {n_layers} Qwen3-30B-A3B layers")
    store, _ = build_layers(QWEN3, n_layers, group, seed=1000)
    dec = HipDecoder(store, DecoderWeights(shape, **decoder_weights(shape)))
    g = torch.Generator(device="cuda")
    g.manual_seed(7000)
    dec.set_lm_head((torch.randn((shape.V, shape.d), generator=g, device="cuda") * 0.02).to(torch.bfloat16))
    dec.weights.t["embed"] = (torch.randn((shape.V, shape.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    dec._w = dec.weights.kernel_w()
    prompt = torch.randint(0, shape.V, (Tp,), generator=g, device="cuda", dtype=torch.int32)
    kvp = KVCacheSet(shape, 1)
    plog = torch.empty(shape.V, dtype=torch.float32, device="cuda")
    dec.prefill_layers(prompt, kvp, 0, plog)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        dec.prefill_layers(prompt, kvp, 0, plog)
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    store.close()
    return {"prompt_tokens": Tp, "layers": n_layers, "reps": reps, "ms": ms, "tok_per_s": Tp / (ms * 1e-3),
            "logits_finite": bool(torch.isfinite(plog).all().item())}


def probe_costs() -> dict:
    """Launch and hand-off costs on this GPU (libjoule_probe.so): a chain of
    dependent one-wave launches on one stream, the same chain replayed from a
    HIP graph, and a launch of nblk blocks with and without the "last block
    finishes" hand-off (release fence + device-scope ticket), per launch."""
    import ctypes

    from joule_amd.build import PROBE_OUT

    if not PROBE_OUT.exists():
        raise ImportError(f"{PROBE_OUT} is missing: build it with `python -m joule_amd.build`")
    P = ctypes.CDLL(str(PROBE_OUT))
    P.jmp_last_error.restype = ctypes.c_char_p
    f = ctypes.c_float()
    tot = ctypes.c_float()

    def chk(rc):
        if rc != 0:
            raise RuntimeError(f"probe failed ({rc}): {P.jmp_last_error().decode()}")

    res = {}
    chk(P.jmp_launch_chain(1000, 0, 5, ctypes.byref(f)))
    res["dependent_launch_us"] = f.value
    chk(P.jmp_launch_chain(64, 1, 50, ctypes.byref(f)))
    res["graph_replayed_launch_us"] = f.value
    ho = {}
    for nblk in (32, 128, 512, 1536):
        chk(P.jmp_handoff(nblk, 1024, 0, 200, ctypes.byref(f), None))
        plain = f.value
        chk(P.jmp_handoff(nblk, 1024, 1, 200, ctypes.byref(f), ctypes.byref(tot)))
        if tot.value != float(nblk * 1024):
            raise RuntimeError(f"hand-off probe sum {tot.value} != {nblk * 1024}")
        ho[str(nblk)] = {"plain_us": plain, "handoff_us": f.value, "handoff_cost_us": f.value - plain}
        log(f"probe: {nblk} blocks, launch {plain:.2f} us, with the hand-off {f.value:.2f} us")
    res["handoff_by_blocks"] = ho
    # the stream ceilings of the B=8 block's two expert kernels: their
    # algorithmic bytes (gate/up and down records of 51.7 routed experts)
    # read by waves of 16 KiB, from HBM
    P.jmp_stream.argtypes = [ctypes.c_ulonglong, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.POINTER(ctypes.c_float)]
    st = {}
    for name, nbytes in (("gateup_86MB", 86 * 1024 * 1024), ("down_43MB", 43 * 1024 * 1024)):
        for wb in (16384, 8192, 4096):
            chk(P.jmp_stream(nbytes, wb, 16, 64, ctypes.byref(f)))
            st[f"{name}_wave{wb // 1024}K"] = {"us": f.value, "GBs": nbytes / (f.value * 1e-6) / 1e9}
            log(f"probe: stream {name}, {wb // 1024} KiB per wave: {f.value:.2f} us "
                f"({nbytes / (f.value * 1e-6) / 1e9:.0f} GB/s)")
    res["stream"] = st
    log(f"probe: dependent launch {res['dependent_launch_us']:.2f} us, graph-replayed "
        f"{res['graph_replayed_launch_us']:.2f} us")
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--layers", type=int, default=16, help="distinct layers the steps rotate over")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--group", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the 48-layer decode step (B=--batch, --steps timed steps); prints its JSON")
    ap.add_argument("--decode-layers", type=int, default=48,
                    help="layers of the --decode-only step (1: every byte of the layer stays in the 256 MB "
                         "Infinity Cache, which shows how much of each kernel's time is HBM bandwidth)")
    ap.add_argument("--kv-f32", action="store_true",
                    help="with --decode-only: float32 caches (the reference's KVCache type) instead of bf16")
    ap.add_argument("--dense-only", action="store_true",
                    help="only a dense model's decode step (Qwen3-8B-shaped, 36 layers) at B=1 and --batch")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 48-layer 512-token prefill (--steps timed passes); prints its JSON")
    ap.add_argument("--zipf-only", action="store_true",
                    help="only the 512-token Zipf-routed block (MFMA branch) on the 16-layer store; prints its JSON")
    ap.add_argument("--plugin-only", action="store_true",
                    help="only the plugin product HipBackend.q4_gemm at T = 1 to 512 (both kernels); prints its JSON")
    ap.add_argument("--probe", action="store_true",
                    help="only the launch and hand-off cost probes (libjoule_probe.so); prints their JSON")
    ap.add_argument("--no-parity", action="store_true",
                    help="skip the comparison of the timed workload with the oracle")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc runs that measure roofline.traffic")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after timing, run 8 torch copies of this many MiB (a known-size kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1.", file=sys.stderr)
        return 2

    # the counter runs first, while this process has not touched the GPU
    only = (args.probe or args.decode_only or args.prefill_only or args.dense_only or args.plugin_only
            or args.zipf_only)
    traffic = None
    if not only and not args.no_traffic:
        traffic = measure_traffic(args.batch, args.group, args.layers)

    import numpy as np
    import torch

    from joule_amd.moe import OLMOE, QWEN3
    from joule_amd.synth import activations

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    if args.probe:
        print(json.dumps({"probe": probe_costs()}), flush=True)
        return 0
    if args.decode_only:
        r = decode_step(args.batch, args.steps, args.warmup, args.group, n_layers=args.decode_layers,
                        kv_f32=args.kv_f32)
        print(json.dumps({"decode_step": r}), flush=True)
        return 0
    if args.prefill_only:
        r = prefill_only(args.group, args.steps)
        print(json.dumps({"prefill_512": r}), flush=True)
        return 0
    if args.dense_only:
        r = {f"B{b}": dense_step(b, args.steps, args.warmup) for b in (1, args.batch)}
        print(json.dumps({"dense_decode": r}), flush=True)
        return 0
    if args.plugin_only:
        print(json.dumps({"plugin_q4_gemm": plugin_q4_gemm(args.group)}), flush=True)
        return 0
    shape, G, B, NL = QWEN3, args.group, args.batch, args.layers
    log(f"building {NL} Qwen3-shaped layers (G={G}) on the GPU")
    store, gw = build_layers(shape, NL, G, seed=1000)
    if args.zipf_only:
        print(json.dumps({"qwen3_zipf512": zipf_block(store, gw, args.steps, NL, check=not args.no_parity)[0]}),
              flush=True)
        return 0
    x_np = activations(B, shape.d)
    x = torch.from_numpy(x_np).cuda()
    log(f"timing B={B}: {args.warmup} warm-up + {args.steps} steps")
    ms, stages, U, dist = measure(store, gw, x, args.steps, args.warmup, NL)
    rb = store.router_bytes_per_weight()
    main_res = block_numbers(shape, G, B, ms, stages, U, args.steps, NL, rb)
    log(f"B={B}: {main_res['tok_per_s']:.0f} tok/s, {ms * 1e3:.1f} us/step, block "
        f"{main_res['block_GBs']:.0f} GB/s, gate/up {main_res['gateup_GBs']:.0f} GB/s, stages {stages}, "
        f"per call {dist}")
    check = not args.no_parity
    parity = {}

    if args.calib_copy_mib > 0:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"ran 8 copies of {args.calib_copy_mib} MiB for counter calibration")

    sweep = {}
    cpu_sweep = {}
    cpu_on = args.cpu_seconds > 0
    cpu_share = args.cpu_seconds / 8.0          # each extra CPU case; the metric's case gets 3 shares
    margins = router_margins(store, NL, x)
    log(f"router margins (p8 - p9) / p8 over {margins['count']} token-layers: min {margins['min']:.3g}, "
        f"{margins['below_1e-4']} below 1e-4")
    gpu_top0 = torch.empty((B, shape.topk), dtype=torch.int32, device="cuda")
    store.layer_ffn_batch(0, x, topk_idx=gpu_top0)
    gpu_top0 = gpu_top0.cpu().numpy()
    moes = oracle_moes(store, gw, NL) if (cpu_on or check) else None
    if check:
        parity[f"qwen3_B{B}"] = block_parity(store, moes, x_np, list(range(NL)))
        log(f"parity qwen3 B={B}: {parity[f'qwen3_B{B}']}")
    xs = {}
    if not args.no_sweep:
        for b in (1, 32):
            xs[b] = activations(b, shape.d)
            xb = torch.from_numpy(xs[b]).cuda()
            m2, st2, U2, d2 = measure(store, gw, xb, max(args.steps // 2, 50), 10, NL)
            r = block_numbers(shape, G, b, m2, st2, U2, max(args.steps // 2, 50), NL, rb)
            sweep[f"qwen3_B{b}"] = {k: r[k] for k in ("tok_per_s", "ms_per_step", "block_GBs", "block_frac",
                                                      "gateup_GBs", "experts_routed_avg")}
            sweep[f"qwen3_B{b}"]["per_call_us"] = d2
            log(f"sweep qwen3 B={b}: {r['tok_per_s']:.0f} tok/s, block {r['block_GBs']:.0f} GB/s, per call {d2}")
            if check:
                sweep[f"qwen3_B{b}"]["parity"] = parity[f"qwen3_B{b}"] = block_parity(store, moes, xs[b],
                                                                                     list(range(NL)))
                log(f"parity qwen3 B={b}: {parity[f'qwen3_B{b}']}")
            if cpu_on:
                cpu_sweep[f"qwen3_B{b}"] = cpu_case(moes, xs[b], cpu_share, f"qwen3 B={b}")[0]

    if not args.no_sweep:
        # the same blocks with 5 activation digit planes (jm_store_set_act_digits):
        # time and error of the precise setting beside the default's
        prec = {}
        store.set_act_digits(5)
        try:
            for b in (B, 1):
                xp_np = x_np if b == B else xs.get(1, activations(1, shape.d))
                xp = torch.from_numpy(xp_np).cuda()
                m5, st5, U5, d5 = measure(store, gw, xp, max(args.steps // 2, 50), 10, NL)
                r5 = block_numbers(shape, G, b, m5, st5, U5, max(args.steps // 2, 50), NL, rb)
                e = {k: r5[k] for k in ("tok_per_s", "ms_per_step", "block_GBs", "block_frac")}
                e["per_call_us"] = d5
                if check:
                    e["parity"] = parity[f"qwen3_B{b}_digits5"] = block_parity(store, moes, xp_np, list(range(NL)))
                prec[f"qwen3_B{b}"] = e
                log(f"5 digits qwen3 B={b}: {r5['tok_per_s']:.0f} tok/s, {m5 * 1e3:.1f} us/step, "
                    f"parity {e.get('parity')}")
        finally:
            store.set_act_digits(0)
        sweep["act_digits_5"] = prec

    if not args.no_sweep:
        sweep["qwen3_zipf512"], gz, xz_np = zipf_block(store, gw, args.steps, NL, check=check)
        if check:
            parity["qwen3_zipf512"] = sweep["qwen3_zipf512"]["parity"]
        if cpu_on:
            zmoes = oracle_moes(store, gz, 1)
            cpu_sweep["qwen3_zipf512"] = cpu_case(zmoes, xz_np, cpu_share, "qwen3 zipf B=512", min_calls=1)[0]
            del zmoes

    cpu = None
    if cpu_on:
        log(f"CPU baseline: oracle restatement, {3 * cpu_share:.0f} s budget for B={B}")
        cpu = cpu_baseline(moes, x_np, 3 * cpu_share, gpu_top0)
        log(f"CPU baseline {cpu['value']:.1f} tok/s on {cpu['cores']} threads, "
            f"top-k equal to the GPU's: {cpu['topk_bitexact_vs_gpu']}")
    del moes

    if not args.no_sweep:
        del store
        torch.cuda.empty_cache()
        # the OLMoE-shaped configurations: the router table left float32 as
        # they state; Q4 groups of 64 (the reference store's and decode
        # kernel's group) and of 32 (the configurations' wording)
        for GO in (64, 32):
            ostore, ogw = build_layers(OLMOE, NL, GO, seed=1000, router_bf16=False)
            omoes = oracle_moes(ostore, ogw, NL) if (cpu_on or check) else None
            sfx = "" if GO == 64 else f"_G{GO}"
            for b in (1, 8):
                key = f"olmoe_B{b}{sfx}"
                xo_np = activations(b, OLMOE.d)
                xb = torch.from_numpy(xo_np).cuda()
                m2, st2, U2, d2 = measure(ostore, ogw, xb, max(args.steps // 2, 50), 10, NL)
                r = block_numbers(OLMOE, GO, b, m2, st2, U2, max(args.steps // 2, 50), NL,
                                  ostore.router_bytes_per_weight())
                sweep[key] = {k: r[k] for k in ("tok_per_s", "ms_per_step", "block_GBs", "block_frac",
                                                "gateup_GBs", "experts_routed_avg")}
                sweep[key].update({"group": GO, "router": "float32"})
                sweep[key]["per_call_us"] = d2
                log(f"sweep {key}: {r['tok_per_s']:.0f} tok/s, block {r['block_GBs']:.0f} GB/s, per call {d2}")
                if check:
                    sweep[key]["parity"] = parity[key] = block_parity(ostore, omoes, xo_np, list(range(NL)))
                    log(f"parity {key}: {parity[key]}")
                if cpu_on:
                    cpu_sweep[key] = cpu_case(omoes, xo_np, cpu_share, key)[0]
            del omoes, ostore
            torch.cuda.empty_cache()
        # the metric's Qwen3 block at Q4 groups of 32 (the configurations'
        # wording; the headline is at the reference store's 64)
        qstore, qgw = build_layers(QWEN3, NL, 32, seed=1000)
        qmoes = oracle_moes(qstore, qgw, NL) if (cpu_on or check) else None
        m2, st2, U2, d2 = measure(qstore, qgw, x, max(args.steps // 2, 50), 10, NL)
        r = block_numbers(QWEN3, 32, B, m2, st2, U2, max(args.steps // 2, 50), NL, qstore.router_bytes_per_weight())
        key = f"qwen3_B{B}_G32"
        sweep[key] = {k: r[k] for k in ("tok_per_s", "ms_per_step", "block_GBs", "block_frac", "gateup_GBs",
                                        "experts_routed_avg")}
        sweep[key].update({"group": 32, "per_call_us": d2})
        log(f"sweep {key}: {r['tok_per_s']:.0f} tok/s, block {r['block_GBs']:.0f} GB/s, per call {d2}")
        if check:
            sweep[key]["parity"] = parity[key] = block_parity(qstore, qmoes, x_np, list(range(NL)))
            log(f"parity {key}: {parity[key]}")
        if cpu_on:
            cpu_sweep[key] = cpu_case(qmoes, x_np, cpu_share, key)[0]
        del qmoes, qstore
        torch.cuda.empty_cache()

    if not args.no_sweep:
        sweep["qwen3_decode48_B8"] = decode_step(8, max(args.steps // 20, 10), 3, G)
        sweep["plugin_q4_gemm"] = plugin_q4_gemm(G)

    if cpu is not None:
        cpu["sweep"] = cpu_sweep
        for k, v in cpu_sweep.items():
            if k in sweep:
                sweep[k]["cpu_tok_per_s"] = v["value"]
                sweep[k]["gpu_over_cpu"] = sweep[k]["tok_per_s"] / v["value"]

    gu_ms = stages["gateup"]
    gate_traffic = block_traffic = None
    if traffic and "block_bytes" in traffic:
        gate_traffic = traffic["bytes"]["k_gateup"]
        block_traffic = traffic["block_bytes"]
        traffic["ratio_to_algorithmic"] = {
            "k_gateup": gate_traffic / main_res["gateup_bytes"],
            "k_down_comb": traffic["bytes"]["k_down_comb"] / main_res["down_bytes"],
            "block": block_traffic / main_res["bytes_alg"]}
        log(f"traffic: block {block_traffic / 1e6:.2f} MB per call against {main_res['bytes_alg'] / 1e6:.2f} MB "
            f"algorithmic, ratios {traffic['ratio_to_algorithmic']}")
    parity_ok = all(v["ok"] for v in parity.values()) if parity else None
    res = {
        "metric": "MoE decode tok/s + achieved HBM GB/s, Qwen3-30B-A3B-shape Q4, B=1 and B=8",
        "value": main_res["tok_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4 weights x 15-bit block-int activations (exact integer group dot), fp32 scale and accumulate",
        "data": "synthetic: N(0,0.02) Q4 experts, bf16-valued router, x~N(0,1), seeded",
        "config": {"workload": f"qwen3-30b-a3b-shaped MoE block, decode B={B}, Q4 group {G}, "
                               f"{NL} rotating layers resident in HBM",
                   "batch": B, "hidden": shape.d, "experts": shape.E, "topk": shape.topk,
                   "intermediate": shape.m, "group": G, "layers_rotated": NL},
        # the target is defined on the whole block: every algorithmic byte of
        # one call (routed experts' records, router table, x in, out) over the
        # event-timed call; the dominant kernel's own ratio sits beside it
        "roofline": {"bound": "hbm", "kernel": "block (router, top-k, k_gateup, k_down_comb)",
                     "achieved": main_res["block_GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": main_res["block_frac"], "traffic": block_traffic,
                     "bytes_per_launch": main_res["bytes_alg"], "avg_launch_ms": ms,
                     "traffic_source": ("rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this workload before the "
                                        "timing (traffic_counters)") if block_traffic else None,
                     "dominant_kernel": {"kernel": "k_gateup", "achieved": main_res["gateup_GBs"],
                                         "frac": main_res["gateup_GBs"] / PEAK_HBM_GBS,
                                         "traffic": gate_traffic, "bytes_per_launch": main_res["gateup_bytes"],
                                         "avg_launch_ms": gu_ms}},
        "block": {k: main_res[k] for k in ("bytes_alg", "block_GBs", "block_frac", "experts_routed_avg",
                                           "down_GBs")},
        "stages_ms": stages,
        "per_call_us": dist,
        "parity": {"ok": parity_ok, "bar_normwise": PARITY_TOL, "configs": parity} if parity else None,
        "traffic_counters": traffic,
        "router_margins": margins,
        "sweep": sweep,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    if parity_ok is False:
        bad = [k for k, v in parity.items() if not v["ok"]]
        log(f"PARITY FAILURE against the oracle in {bad}: the numbers above are not valid")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
