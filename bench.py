"""Benchmark of the quantized decode hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): the binary sign-plane organ
(512x2048, 1 bit/weight + f16 mean|w| per 128) streamed over many distinct
organs in ONE launch, working set > 1 GB (so the 256 MB MALL cannot serve
repeats), inputs resident in HBM.  A "step" is one launch over all organs.
Every timed loop is preceded by about 0.2 s of untimed launches of the same
work (the GPU clocks ramp up over the first milliseconds of activity), then
the W warmup steps, then exactly K timed steps between HIP events.

Also reported (the same JSON line, "extra"): Q4 (config 1), mixed, q8,
HGRAVS01 low-rank and HGRAVR02 streamed GB/s, the binary down shape
(2048x512), the terminal head, single-organ latency, the config-3 MoE layer,
the config-4 48-layer mixed token (per-layer launches, and as one persistent
launch) and the mixed-1p5-v1 48-layer token (the reference's own codec
triplet) in microseconds at batch 1, and the config-5 batched block.

The CPU baseline is the oracle's serial restatement of
binary_group_matvec_f32 (crates/hawking-core/src/model/qwen_complete_binary/
q80_mixed_decode.rs:245-257) on a bounded sample of the same organs, one
thread, timed on this host; "extra.cpu_baselines" times the oracle on the
other configs the same way (c1 Q4 organ, c3 layer, c4 token from a sample of
layers, c5 block from a sample of tokens) and the c2 organ on every host
thread.  `--only NAME` runs one workload and prints its result (for
profiler runs).  The headline and the decode tokens also carry per-call
distributions (median, p10, p90 of 100 calls, each between its own pair of
HIP events).

roofline.traffic (HBM bytes per headline launch) is measured in the run:
after the timed work, two child rocprofv3 --pmc passes (FETCH_SIZE, then
WRITE_SIZE) run the headline workload, each counter scaled by what it reads
for a 512 MiB device copy in the same pass ("extra.traffic_measurement");
only if the profiler is absent or a pass fails does the committed summary
under profiles/ stand in, and the line says so.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
SEED = 0x48415752
HK_Q4, HK_BIN, HK_MIXED, HK_F32, HK_Q8, HK_U3, HK_BIN_RICE = 0, 1, 2, 3, 4, 5, 6
WORKLOADS = {
    # name: (kind, group, rows, cols, n_organs)
    "binary_512x2048": (HK_BIN, 128, 512, 2048, 8192),
    "binary_2048x512": (HK_BIN, 128, 2048, 512, 8192),
    "q4g32_512x2048": (HK_Q4, 32, 512, 2048, 2048),
    "mixed_512x2048": (HK_MIXED, 128, 512, 2048, 8192),
    "q8g64_512x2048": (HK_Q8, 64, 512, 2048, 1024),
    "binary_rice_512x2048": (HK_BIN_RICE, 128, 512, 2048, 4096),
}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def organ_stream_id(workload: str, i: int) -> int:
    return (0xBE << 48) | (sorted(WORKLOADS).index(workload) << 40) | i


def build_stream(ctx, name: str, n_organs: int | None = None):
    from hawking_amd import organs
    kind, group, rows, cols, n = WORKLOADS[name]
    n = n_organs or n
    orgs = []
    for i in range(n):
        sid = organ_stream_id(name, i)
        orgs.append(organs.SyntheticOrgan(ctx, kind, rows, cols, organs.stream_key(SEED, sid),
                                          organs.stream_key(SEED, sid ^ (1 << 47)), group=group))
    oset = organs.OrganSet(ctx, orgs)
    x = ctx.empty((n, cols))
    from hawking_amd.organs import stream_key
    ctx.call("hk_synth_normal", stream_key(SEED, 0xBE0001), 0, n * cols, 1.0, x.ptr, ctx.stream)
    y = ctx.empty((n, rows))
    alg_bytes = oset.packed_bytes + n * (rows + cols) * 4
    return oset, x, y, alg_bytes


RAMP_S = 0.2  # seconds of untimed launches before each timed loop (--ramp)


def time_launches(ctx, fn, steps: int, warmup: int, ramp_s: float | None = None) -> float:
    """Average ms per call of fn() over `steps` calls, HIP events on ctx.stream,
    after ramp_s seconds of untimed calls and `warmup` more."""
    t_end = time.perf_counter() + (RAMP_S if ramp_s is None else ramp_s)
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        ctx.synchronize()
    for _ in range(warmup):
        fn()
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    ctx.synchronize()
    return e0.elapsed_ms(e1) / steps


def launch_distribution(ctx, fn, reps: int = 100, warmup: int = 5) -> dict:
    """Per-call times of `reps` back-to-back calls of fn(), each between its
    own pair of HIP events on ctx.stream (one event between consecutive
    calls): median, p10 and p90 in ms."""
    for _ in range(warmup):
        fn()
    ev = [ctx.event() for _ in range(reps + 1)]
    ctx.synchronize()
    ev[0].record()
    for i in range(reps):
        fn()
        ev[i + 1].record()
    ctx.synchronize()
    t = np.array([ev[i].elapsed_ms(ev[i + 1]) for i in range(reps)])
    return {"reps": reps, "median_ms": round(float(np.median(t)), 5), "p10_ms": round(float(np.percentile(t, 10)), 5),
            "p90_ms": round(float(np.percentile(t, 90)), 5)}


def streamed(ctx, name, steps, warmup, n_organs=None):
    oset, x, y, nbytes = build_stream(ctx, name, n_organs)
    kind, group, rows, cols, _ = WORKLOADS[name]
    ms = time_launches(ctx, lambda: oset.gemv(x, cols, y, rows), steps, warmup)
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9, "organs": len(oset.organs),
            "packed_bytes_per_organ": oset.packed_bytes / len(oset.organs)}, (oset, x, y)


def lowrank_streamed(ctx, steps, warmup, rows=2048, rank=160, cols=768, n=4096):
    """HGRAVS01 r160 (3-bit factors) as the routed down_proj shape: n low-rank
    organs, y_i = L_i (R_i x_i) for all i in one launch (hk_gemv_lowrank_set:
    one workgroup per pair, mid kept on chip).  Algorithmic bytes: the
    canonical packed factors plus x and y."""
    from hawking_amd import organs
    lefts, rights = [], []
    for i in range(n):
        sid = (0xB5 << 48) | i
        lefts.append(organs.SyntheticOrgan(ctx, HK_U3, rows, rank, organs.stream_key(SEED, sid), 0, group=64,
                                           sigma=0.05))
        rights.append(organs.SyntheticOrgan(ctx, HK_U3, rank, cols, organs.stream_key(SEED, sid ^ (1 << 47)), 0,
                                            group=64))
    ls, rs = organs.OrganSet(ctx, lefts), organs.OrganSet(ctx, rights)
    x = ctx.empty((n, cols))
    ctx.call("hk_synth_normal", organs.stream_key(SEED, 0xB50001), 0, n * cols, 1.0, x.ptr, ctx.stream)
    y = ctx.empty((n, rows))

    def step():
        organs.gemv_lowrank_set(ctx, ls, rs, x, cols, y, rows)

    ms = time_launches(ctx, step, steps, warmup)
    nbytes = ls.packed_bytes + rs.packed_bytes + n * (cols + rows) * 4
    return {"gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "us_per_step": round(ms * 1e3, 1), "organs": n, "shape": [rows, rank, cols],
            "packed_bytes_per_organ": round((ls.packed_bytes + rs.packed_bytes) / n, 1)}


def terminal_head_bench(ctx, steps, warmup, vocab=151936, hidden=2048, n_valid=151669):
    """The device terminal head on the Qwen80 shape: final RMSNorm(1+w), a
    synthetic q8 G64 lm_head (vocab x hidden), greedy token on the device."""
    from hawking_amd import organs
    from hawking_amd.head import TerminalHead
    lm = organs.SyntheticOrgan(ctx, HK_Q8, vocab, hidden, organs.stream_key(SEED, 0xEAD0), 0, group=64, sigma=0.02)
    nw = np.zeros(hidden, np.float32)
    head = TerminalHead(ctx, nw, lm, n_valid)
    hs = ctx.empty((4, hidden))
    ctx.call("hk_synth_normal", organs.stream_key(SEED, 0xEAD1), 0, 4 * hidden, 1.0, hs.ptr, ctx.stream)
    state = {"i": 0}

    def step():
        head.greedy_device(hs.offset(hidden * (state["i"] % 4)))
        state["i"] += 1

    ms = time_launches(ctx, step, steps, warmup)
    nbytes = lm.packed_bytes + hidden * 4 * 3 + vocab * 4
    return {"us_per_token": round(ms * 1e3, 2), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "lm_head_bytes": lm.packed_bytes,
            "shape": [vocab, hidden], "n_valid": n_valid}


def moe15_bench(ctx, steps, warmup, n_layers=48, H=2048, I=512, SI=512, E=512, K=10, rank=160, n_inputs=16):
    """The mixed-1p5-v1 token's MoE suffixes at batch 1 (config-4 shape,
    Qwen3-Next-80B-A3B): per layer 512 experts with an HGRAVB01 gate, an
    HGRAVR02 up (2% Rice residual) and an HGRAVS01 r160 3-bit down; q8
    router, shared-expert gate and shared expert.  Tokens cycle over
    n_inputs distinct hidden vectors (distinct routes).  Algorithmic bytes per
    token: the canonical packed bytes of every organ the routes touch, the
    norm weights and the hidden state in and out."""
    from hawking_amd import organs
    from hawking_amd.moe import Mixed15Dims, mixed15_decode_stack, synthetic_mixed15_layers
    t0 = time.time()
    layers, expert_bytes, dense_bytes = synthetic_mixed15_layers(ctx, SEED, n_layers,
                                                                 Mixed15Dims(H, I, SI, E, K, rank))
    ctx.synchronize()
    gen_s = time.time() - t0
    hs = ctx.empty((n_inputs, H))
    ctx.call("hk_synth_normal", organs.stream_key(SEED, 0xBE0015), 0, n_inputs * H, 1.0, hs.ptr, ctx.stream)
    out = ctx.empty(H)
    ids = ctx.empty((n_inputs, n_layers, K), np.int32)
    state = {"i": 0}

    def step():
        i = state["i"] % n_inputs
        state["i"] += 1
        mixed15_decode_stack(ctx, layers, hs.offset(i * H), out, ids.offset(i * n_layers * K))

    ctx.device_status()
    ms = time_launches(ctx, step, steps, warmup)
    status = ctx.device_status()
    dist = launch_distribution(ctx, step, 100)
    routes = ids.download()
    per_tok = [sum(dense_bytes[l] + 2 * H * 4 + sum(expert_bytes[l][int(e)] for e in routes[t, l])
                   for l in range(n_layers)) for t in range(n_inputs)]
    tok_bytes = float(np.mean(per_tok))
    return {"us_per_token": round(ms * 1e3, 2), "bytes_per_token": round(tok_bytes),
            "gbps": round(tok_bytes / (ms * 1e-3) / 1e9, 1), "tokens_per_s": round(1e3 / ms, 1),
            "launches_per_layer": 4, "layers": n_layers, "device_status": status,
            "distinct_routes": int(np.unique(routes.reshape(-1, K), axis=0).shape[0]), "gen_seconds": round(gen_s, 2),
            "per_call_us": {"median": round(dist["median_ms"] * 1e3, 2), "p10": round(dist["p10_ms"] * 1e3, 2),
                            "p90": round(dist["p90_ms"] * 1e3, 2), "reps": dist["reps"]}}


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def token_cache_label(r):
    """Whether a token's bytes can stay in the Infinity Cache between the
    tokens that cycle over them: a layer's weights are read again only after
    the whole token's other bytes went through."""
    b = r["bytes_per_token"]
    if b > MALL_BYTES:
        r["cache"] = (f"MALL-cold ({b / 1e6:.0f} MB read per token, more than the 256 MB Infinity Cache, "
                      f"before a layer's weights are read again)")
    else:
        r["cache"] = f"MALL-warm ({b / 1e6:.0f} MB read per token fits the 256 MB Infinity Cache)"
    return r


def stream_control(ctx, steps, warmup, nbytes=4 << 30, workgroup_counts=(1024, 2048, 4096, 8192)):
    """The achievable-bandwidth control (hk_stream_control): one read of a
    4 GiB buffer (16 x the MALL) per launch with 16-byte loads, at several
    workgroup counts; the best is this box's read ceiling under the same
    timing as the organ GEMVs."""
    buf = ctx.empty(nbytes, np.uint8)
    ctx.call("hk_memset", buf.ptr, 0x3C, nbytes, ctx.stream)
    out = ctx.empty(max(workgroup_counts))
    rates = {}
    for wg in workgroup_counts:
        ms = time_launches(ctx, lambda: ctx.call("hk_stream_control", buf.ptr, nbytes, out.ptr, wg, ctx.stream),
                           steps, warmup)
        rates[wg] = nbytes / (ms * 1e-3) / 1e9
    best = max(rates, key=rates.get)
    return {"gbps": round(rates[best], 1), "frac_hbm": round(rates[best] / HBM_PEAK_GBPS, 4), "workgroups": best,
            "bytes": nbytes, "gbps_by_workgroups": {str(k): round(v, 1) for k, v in rates.items()}}


def single_organ_us(ctx, steps=200):
    from hawking_amd import organs
    o = organs.SyntheticOrgan(ctx, HK_BIN, 512, 2048, organs.stream_key(SEED, 0xBE0002))
    x = ctx.empty(2048)
    ctx.call("hk_synth_normal", organs.stream_key(SEED, 0xBE0003), 0, 2048, 1.0, x.ptr, ctx.stream)
    y = ctx.empty(512)
    return time_launches(ctx, lambda: o.matvec_device(x, y), steps, 20) * 1e3


def moe_bench(ctx, shape, steps, warmup, n_inputs=16, persistent=False):
    """Decode `steps` tokens cycling over n_inputs distinct hidden vectors
    (distinct routings, so the MALL does not serve repeated experts).
    persistent: the token as one persistent launch (HK_STACK_PERSISTENT)
    instead of the per-layer launches."""
    from hawking_amd.moe import MoeModel
    from hawking_amd.organs import stream_key
    t0 = time.time()
    m = MoeModel(ctx, shape)
    m.fill_synthetic(SEED)
    if persistent:
        m.set_stack_launch(1)
        if not m.stack_is_persistent():
            raise RuntimeError("the persistent launch is not admitted for this shape")
    ctx.synchronize()
    gen_s = time.time() - t0
    H, L, K = shape.hidden, shape.n_layers, shape.top_k
    hs = ctx.empty((n_inputs, H))
    ctx.call("hk_synth_normal", stream_key(SEED, 0xBE0004), 0, n_inputs * H, 1.0, hs.ptr, ctx.stream)
    out = ctx.empty(H)
    ids = ctx.empty((n_inputs, L, K), np.int32)
    state = {"i": 0}

    def step():
        i = state["i"] % n_inputs
        state["i"] += 1
        m.decode_stack_device(hs.offset(i * H), out, ids.offset(i * L * K), None)

    ms = time_launches(ctx, step, steps, warmup)
    dist = launch_distribution(ctx, step, 100)
    # algorithmic bytes per token from the routes actually taken
    routes = ids.download()
    dev_bytes, dense_per_layer = m.model_bytes()
    per_tok = []
    for t in range(n_inputs):
        b = 0
        for layer in range(L):
            b += dense_per_layer + 2 * H * 4
            for e in routes[t, layer]:
                b += m.expert_bytes(layer, int(e))
            if shape.shared_inter:
                b += m.expert_bytes(layer, shape.n_experts)
        per_tok.append(b)
    tok_bytes = float(np.mean(per_tok))
    return {"us_per_token": ms * 1e3, "bytes_per_token": tok_bytes, "gbps": tok_bytes / (ms * 1e-3) / 1e9,
            "model_device_bytes": dev_bytes, "gen_seconds": round(gen_s, 2), "layers": L,
            "per_call_us": {"median": round(dist["median_ms"] * 1e3, 2), "p10": round(dist["p10_ms"] * 1e3, 2),
                            "p90": round(dist["p90_ms"] * 1e3, 2), "reps": dist["reps"]}}


def moe_layer_cold_bench(ctx, steps, warmup, n_layers=16, n_inputs=16):
    """Config 3's layer with the MALL defeated: a 16-layer model of c3 layers
    (distinct weights), step i runs layer i % 16 on input i % 16, so the
    bytes a step touches (about 24 MB) were last read 16 steps (about
    380 MB of other layers' data) earlier."""
    from hawking_amd.moe import MoeModel, MoeShape
    from hawking_amd.organs import stream_key
    shape = MoeShape(n_layers=n_layers, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                     expert_kind=HK_Q4, expert_group=32)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(SEED)
    H, K = shape.hidden, shape.top_k
    hs = ctx.empty((n_inputs, H))
    ctx.call("hk_synth_normal", stream_key(SEED, 0xBE0005), 0, n_inputs * H, 1.0, hs.ptr, ctx.stream)
    out = ctx.empty(H)
    ids = ctx.empty((n_layers * n_inputs, K), np.int32)
    state = {"i": 0}

    def step():
        i = state["i"]
        state["i"] += 1
        m.decode_layer_device(i % n_layers, hs.offset((i % n_inputs) * H), out,
                              ids.offset(((i % n_layers) * n_inputs + (i // n_layers) % n_inputs) * K), None)

    ms = time_launches(ctx, step, max(steps, 64), warmup)
    routes = ids.download()
    _, dense_per_layer = m.model_bytes()
    per = [dense_per_layer + 2 * H * 4 + sum(m.expert_bytes(l, int(e)) for e in routes[l * n_inputs + j])
           + m.expert_bytes(l, shape.n_experts) for l in range(n_layers) for j in range(n_inputs)]
    nbytes = float(np.mean(per))
    return {"us_per_layer": round(ms * 1e3, 2), "bytes_per_layer": round(nbytes), "gbps": round(nbytes / ms / 1e6, 1),
            "cache": "MALL-cold (16 distinct layers cycled)"}


PMC_CALIB_MB = 512


def _pmc_pass(counter: str, timeout_s: float):
    """One rocprofv3 --pmc pass over a child run of the headline workload
    (--only-main, no ramp, 1 warm-up and 3 timed launches, after a 512 MiB
    device copy): the mean KiB per headline dispatch of `counter` and the KiB
    the copy read (FETCH_SIZE) or wrote (WRITE_SIZE).  Raises on failure."""
    import glob
    import shutil
    import signal
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        raise RuntimeError("rocprofv3 not found")
    d = tempfile.mkdtemp(prefix="hk_pmc_", dir="/tmp")
    try:
        # the profiled program itself after "--" (no launcher in between)
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--", sys.executable,
               os.path.abspath(__file__), "--only-main", "--no-cpu", "--ramp", "0", "--steps", "3", "--warmup", "1",
               "--calib-copy-mb", str(PMC_CALIB_MB)]
        env = dict(os.environ, TMPDIR="/tmp")
        p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                             start_new_session=True)
        try:
            rc = p.wait(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            raise RuntimeError(f"{counter} pass timed out")
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise RuntimeError(f"{counter} pass wrote no counter file (exit {rc})")
        return pmc_headline_and_copy(files, counter, f"exit {rc}")
    finally:
        shutil.rmtree(d, ignore_errors=True)


def pmc_headline_and_copy(files, counter: str, note: str = ""):
    """From rocprofv3 counter-collection CSV files: `counter` summed over its
    dimensions per dispatch, then the mean over the headline GEMV's
    dispatches (gemv_tiled_kernel, at least 3) and the largest copy
    dispatch (the calibration copy).  Raises if either is missing."""
    import csv
    per_dispatch = {}
    for fn in files:
        with open(fn, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                key = (fn, row.get("Dispatch_Id"))
                name, v = per_dispatch.get(key, (row.get("Kernel_Name", ""), 0.0))
                per_dispatch[key] = (name, v + float(row["Counter_Value"]))
    gemv = [v for name, v in per_dispatch.values() if "gemv_tiled_kernel" in name]
    copies = [v for name, v in per_dispatch.values() if "copy" in name.lower()]
    if len(gemv) < 3 or not copies:
        raise RuntimeError(f"{counter} pass: {len(gemv)} headline and {len(copies)} copy dispatches ({note})")
    return sum(gemv) / len(gemv), max(copies)


def live_traffic(timeout_s: float = 240.0):
    """HBM bytes per launch of the headline kernel, measured in this run: two
    rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE) over a child run of
    the same workload, each counter scaled by what it reads for a 512 MiB
    device copy in that pass.  Returns (bytes, details) or (None, reason)."""
    try:
        fk, fc = _pmc_pass("FETCH_SIZE", timeout_s)
        wk, wc = _pmc_pass("WRITE_SIZE", timeout_s)
    except Exception as e:  # noqa: BLE001 -- reported in the line, the committed summary stands in
        return None, str(e)
    copy_kib = PMC_CALIB_MB * 1024.0
    ff, wf = copy_kib / fc, copy_kib / wc
    return int(round((fk * ff + wk * wf) * 1024)), {
        "fetch_size_kib_per_dispatch": round(fk, 1), "write_size_kib_per_dispatch": round(wk, 1),
        "calibration_copy_bytes": PMC_CALIB_MB << 20, "calibration_fetch_size_kib": round(fc, 1),
        "calibration_write_size_kib": round(wc, 1), "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}


def measured_traffic(workload: str):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (each counter scaled by what it reads for a
    512 MiB device copy); None if no summary for this workload is present.
    Used when the run's own counter passes cannot be made (live_traffic)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"gemv_{workload}_streamed.pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        pmc = json.load(f)
    if pmc.get("workload") != workload:
        return None
    return int(round((pmc["fetch_size_kib_per_dispatch"] * pmc["fetch_factor"] +
                      pmc["write_size_kib_per_dispatch"] * pmc["write_factor"]) * 1024))


def moe_batch_bench(ctx, steps, warmup, n_batches=8, T=32):
    """Config 5: the DeepSeek-V3-shaped noaux_tc block on batches of T bf16
    tokens, cycling over n_batches distinct batches (distinct routings)."""
    from hawking_amd.moe import MoeModel, MoeShape
    from hawking_amd.organs import stream_key
    shape = MoeShape.deepseek_v3()
    t0 = time.time()
    m = MoeModel(ctx, shape)
    m.fill_synthetic(SEED)
    ctx.synchronize()
    gen_s = time.time() - t0
    H, K = shape.hidden, shape.top_k
    xf = ctx.empty((n_batches, T, H))
    ctx.call("hk_synth_normal", stream_key(SEED, 0xC5C5), 0, n_batches * T * H, 1.0, xf.ptr, ctx.stream)
    x32 = xf.download()
    b = x32.view(np.uint32).astype(np.uint64)
    xb = ctx.to_device(((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16))  # bf16, round to nearest even
    y = ctx.empty((T, H))
    ids = ctx.empty((n_batches, T, K), np.int32)
    state = {"i": 0}

    def step():
        i = state["i"] % n_batches
        state["i"] += 1
        m.forward_batch_device(0, xb.offset(i * T * H), T, y, ids.offset(i * T * K), None)

    ms = time_launches(ctx, step, steps, warmup)
    routes = ids.download()
    dev_bytes, dense_per_layer = m.model_bytes()
    router_bytes = shape.n_experts * H * 4 + shape.n_experts * 4
    shared_bytes = m.expert_bytes(0, shape.n_experts)
    per_batch, active = [], []
    for bi in range(n_batches):
        experts = sorted(set(int(e) for e in routes[bi].ravel()))
        active.append(len(experts))
        per_batch.append(router_bytes + sum(m.expert_bytes(0, e) for e in experts) + shared_bytes + T * H * (2 + 4))
    nbytes = float(np.mean(per_batch))
    return {"us_per_step": ms * 1e3, "tokens_per_step": T, "tokens_per_s": T / (ms * 1e-3),
            "bytes_per_step": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9,
            "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, "active_experts_mean": float(np.mean(active)),
            "model_device_bytes": dev_bytes, "gen_seconds": round(gen_s, 2)}


def cpu_baseline(budget_s: float = 12.0, n_distinct: int = 64):
    """Oracle binary matvec (serial f32, one thread) over the first n_distinct
    organs of the headline workload, cycled until budget_s of matvec time."""
    from oracle import hk_oracle as oracle
    kind, group, rows, cols, _ = WORKLOADS["binary_512x2048"]
    per_organ = 147_456 + (rows + cols) * 4
    xkey = oracle.stream_key(SEED, 0xBE0001)
    organs = []
    for i in range(n_distinct):
        sid = organ_stream_id("binary_512x2048", i)
        w = oracle.normal(oracle.stream_key(SEED, sid), rows * cols, 0.02).reshape(rows, cols)
        s, g = oracle.bin_pack(w)
        organs.append((s, g, oracle.normal(xkey, cols, 1.0, first=i * cols)))
    done, t_total = 0, 0.0
    while t_total < budget_s:
        s, g, x = organs[done % n_distinct]
        t0 = time.perf_counter()
        oracle.bin_matvec(s, g, rows, cols, x)
        t_total += time.perf_counter() - t0
        done += 1
    return {"value": round(done * per_organ / t_total / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{done} matvecs cycling over {n_distinct} distinct binary 512x2048 organs of the headline "
                      f"workload (9.4 MB, cache-resident on the CPU): the oracle's serial f32 restatement of "
                      f"binary_group_matvec_f32, 1 thread, {t_total:.1f} s",
            **host_info()}


def host_info() -> dict:
    """The host CPU (model, threads this process may use) and the oracle's compiler and flags."""
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    except (OSError, IndexError):
        cc = "gcc (version unknown)"
    return {"cpu_model": model, "host_threads": len(os.sched_getaffinity(0)), "compiler": cc,
            "flags": "-O2 -std=c11 -ffp-contract=off -fno-fast-math"}


def cpu_baselines(budget_s: float = 3.0) -> dict:
    """The oracle on the other configs, each on a bounded sample (about
    budget_s of timed work after building the sample), one thread unless
    stated.  Weights are the same draws the device generates."""
    from oracle import hk_oracle as oracle
    from tests import hk_testutil as U
    from hawking_amd.moe import MoeShape
    out = {}

    def timed(fn, budget=budget_s):
        n, t = 0, 0.0
        while t < budget:
            t0 = time.perf_counter()
            fn()
            t += time.perf_counter() - t0
            n += 1
        return t / n

    # c1: one Q4 G32 organ 512x2048 (the workload's first organ)
    sid = organ_stream_id("q4g32_512x2048", 0)
    w = oracle.normal(oracle.stream_key(SEED, sid), 512 * 2048, 0.02).reshape(512, 2048)
    s, c = oracle.q4_pack(w, 32)
    x = oracle.normal(oracle.stream_key(SEED, 0xBE0001), 2048, 1.0)
    sec = timed(lambda: oracle.q4_matvec(s, c, 512, 2048, 32, x))
    out["c1_q4g32_512x2048"] = {"us_per_organ": round(sec * 1e6, 1), "gbps": round(600_064 / sec / 1e9, 4),
                                "cores": 1, "sample": "Qwen80Q4PackedTensor::matvec restated, one organ, repeated"}
    # c2 on every host thread: whole organs per thread (each keeps the serial row order)
    nt = len(os.sched_getaffinity(0))
    orgs = []
    for i in range(4 * nt):
        sid = organ_stream_id("binary_512x2048", i)
        w = oracle.normal(oracle.stream_key(SEED, sid), 512 * 2048, 0.02).reshape(512, 2048)
        orgs.append(oracle.bin_pack(w) + (oracle.normal(oracle.stream_key(SEED, 0xBE0001), 2048, 1.0, first=i * 2048),))
    with cf.ThreadPoolExecutor(max_workers=nt) as pool:
        def wave():
            list(pool.map(lambda o: oracle.bin_matvec(o[0], o[1], 512, 2048, o[2]), orgs))
        sec = timed(wave)
    out["c2_binary_512x2048_all_threads"] = {"gbps": round(len(orgs) * 157_696 / sec / 1e9, 4), "cores": nt,
                                             "sample": f"{len(orgs)} distinct organs per wave over {nt} threads"}
    # c3 and c4: moe_suffix of sampled layers (the oracle regenerates the routed and shared experts)
    cache = {}
    with cf.ThreadPoolExecutor(max_workers=nt) as pool:
        for label, kind, group, layers in (("c3_qwen3next_layer_q4", HK_Q4, 32, 1),
                                           ("c4_48_layer_token_mixed", HK_MIXED, 128, 3)):
            shape = MoeShape(n_layers=48, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                             expert_kind=kind, expert_group=group)
            h = oracle.normal(oracle.stream_key(SEED, 0xBE0004), 2048, 1.0)
            per_layer = []
            for layer in range(layers):
                cache.clear()
                L, h2, *_ = U.oracle_layer_cached(oracle, SEED, shape, layer, h, cache, pool)
                per_layer.append(timed(lambda: L.forward(h), budget_s / layers))
                h = h2
            mean = float(np.mean(per_layer))
            if layers == 1:
                out[label] = {"us_per_layer": round(mean * 1e6, 1), "cores": 1,
                              "sample": "moe_suffix restated (f32 router, top-10, 10 routed + shared Q4 experts)"}
            else:
                out[label] = {"ms_per_token": round(mean * 48 * 1e3, 2), "cores": 1,
                              "sample": f"48 x the mean moe_suffix time of layers 0..{layers - 1} (mixed experts)"}
        # c5: routed_moe per token on sampled tokens; a batch of 32 = 32 tokens
        shape = MoeShape.deepseek_v3()
        xs = oracle.normal(oracle.stream_key(SEED, 0xC5C5), 2 * 7168, 1.0).reshape(2, 7168)
        per_tok = []
        for t in range(2):
            xb = U.bf16_to_f32(U.to_bf16_bits(xs[t]))
            M, *_ = _oracle_noaux_pooled(oracle, U, shape, xb, pool)
            per_tok.append(timed(lambda: M.forward(xb), budget_s / 2))
        out["c5_dsv3_block_32_tokens"] = {"ms_per_step": round(float(np.mean(per_tok)) * 32 * 1e3, 1), "cores": 1,
                                          "sample": "32 x the mean routed_moe time of 2 tokens (8 routed + shared "
                                                    "Q4 experts each, f32 router, noaux_tc)"}
    return out


def _oracle_noaux_pooled(oracle, U, shape, x, pool):
    """U.oracle_noaux with the experts generated on a thread pool."""
    _, router, _ = U.dense(oracle, SEED, shape, 0)
    bias = U.router_bias(oracle, SEED, shape, 0)
    logits = oracle.gemv_f32(router, x)
    ids, _ = oracle.router_noaux_tc(logits, bias, shape.n_group, shape.topk_group, shape.top_k,
                                    shape.norm_topk_prob, shape.routed_scaling_factor)
    want = [int(e) for e in ids] + [shape.n_experts]
    made = list(pool.map(lambda ep: U.oracle_organ(oracle, SEED, shape, 0, ep[0], ep[1]),
                         [(e, p) for e in want for p in range(3)]))
    experts = [None] * shape.n_experts
    for i, e in enumerate(want[:-1]):
        experts[e] = tuple(made[3 * i:3 * i + 3])
    M = oracle.NoauxMoe(shape.hidden, shape.n_experts, shape.top_k, shape.n_group, shape.topk_group,
                        shape.norm_topk_prob, shape.routed_scaling_factor, router, bias, experts, tuple(made[-3:]))
    return M, ids


def spot_check(ctx, oset, x, y, n_check=4):
    """GPU output of the first organs of the timed set vs the oracle."""
    from oracle import hk_oracle as oracle
    kind, group, rows, cols, _ = WORKLOADS["binary_512x2048"]
    yg = y.download()
    xs = x.download()
    worst = 0.0
    for i in range(n_check):
        sid = organ_stream_id("binary_512x2048", i)
        w = oracle.normal(oracle.stream_key(SEED, sid), rows * cols, 0.02).reshape(rows, cols)
        s, g = oracle.bin_pack(w)
        xi = oracle.normal(oracle.stream_key(SEED, 0xBE0001), cols, 1.0, first=i * cols)
        assert np.array_equal(xi, xs[i]), "device input generator disagrees with the oracle"
        worst = max(worst, oracle.relative_l2(yg[i], oracle.bin_matvec(s, g, rows, cols, xs[i])))
    return worst


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only-main", action="store_true", help="headline kernel only (for profiling)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--moe15-only", action="store_true", help="only the mixed-1p5-v1 token (development)")
    ap.add_argument("--only", default="", help="run one named workload and print its result (profiling)")
    ap.add_argument("--moe-layers", type=int, default=48)
    ap.add_argument("--ramp", type=float, default=0.2,
                    help="seconds of untimed launches before each timed loop (0 under counter collection)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="run one device-to-device copy of this size first (PMC byte-counter calibration)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="take roofline.traffic from the committed summary instead of two rocprofv3 --pmc passes")
    args = ap.parse_args()
    global RAMP_S
    RAMP_S = args.ramp
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path: organ GEMVs would shard by rows, MoE layers by experts)", file=sys.stderr)
        sys.exit(2)

    from hawking_amd.runtime import Context
    ctx = Context(0)
    info = ctx.device_info()
    log("device", info)
    if args.calib_copy_mb:
        nb = args.calib_copy_mb << 20
        src, dst = ctx.empty(nb, np.uint8), ctx.empty(nb, np.uint8)
        ctx.call("hk_memset", src.ptr, 1, nb, ctx.stream)
        ctx.call("hk_memcpy_dtod", dst.ptr, src.ptr, nb, ctx.stream)
        ctx.synchronize()
        log("calibration copy bytes", nb)
        del src, dst

    if args.moe15_only:
        r = moe15_bench(ctx, max(args.steps, 20), args.warmup, n_layers=args.moe_layers)
        log("mixed-1p5 token", r)
        print(json.dumps({"moe15_token_c4_mixed_1p5_v1": r}), flush=True)
        return

    from hawking_amd.moe import MoeShape
    c3 = MoeShape(n_layers=1, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                  expert_kind=HK_Q4, expert_group=32)
    c4 = MoeShape(n_layers=args.moe_layers, hidden=2048, inter=512, shared_inter=512, n_experts=512,
                  top_k=10, expert_kind=HK_MIXED, expert_group=128)
    tok_steps = max(args.steps, 20)

    def streamed_extra(name):
        r, bufs = streamed(ctx, name, args.steps, args.warmup)
        del bufs
        return {"gbps": round(r["gbps"], 1), "frac_hbm": round(r["gbps"] / HBM_PEAK_GBPS, 4),
                "us_per_launch": round(r["ms"] * 1e3, 1), "organs": r["organs"],
                "packed_bytes_per_organ": round(r["packed_bytes_per_organ"], 1)}

    def rounded(r, nd=2):
        return {k: (round(v, nd) if isinstance(v, float) else v) for k, v in r.items()}

    workloads = {name: (lambda n=name: streamed_extra(n)) for name in
                 ("binary_2048x512", "q4g32_512x2048", "mixed_512x2048", "q8g64_512x2048", "binary_rice_512x2048")}
    workloads.update({
        "stream_control_read_4gib": lambda: stream_control(ctx, args.steps, args.warmup),
        "hgravs01_r160_2048x768": lambda: lowrank_streamed(ctx, args.steps, args.warmup),
        "terminal_head_q8_151936x2048": lambda: terminal_head_bench(ctx, tok_steps, args.warmup),
        "single_organ_binary_512x2048_us": lambda: round(single_organ_us(ctx), 2),
    })
    moe_workloads = {
        "moe_layer_c3_q4": lambda: dict(rounded(moe_bench(ctx, c3, tok_steps, args.warmup)),
                                        cache="MALL-warm (one layer, 16 inputs: about 24 MB per token, "
                                              "all within the 256 MB Infinity Cache)"),
        "moe_layer_c3_q4_cold": lambda: moe_layer_cold_bench(ctx, tok_steps, args.warmup),
        "moe_token_c4_mixed": lambda: token_cache_label(rounded(moe_bench(ctx, c4, tok_steps, args.warmup))),
        "moe_token_c4_mixed_persistent": lambda: token_cache_label(
            rounded(moe_bench(ctx, c4, tok_steps, args.warmup, persistent=True))),
        "moe15_token_c4_mixed_1p5_v1": lambda: token_cache_label(
            moe15_bench(ctx, tok_steps, args.warmup, n_layers=args.moe_layers)),
        "moe_batch_c5_dsv3": lambda: rounded(moe_batch_bench(ctx, max(args.steps, 10), args.warmup), 4),
    }
    if args.only:
        table = dict(workloads, **moe_workloads)
        if args.only not in table and args.only not in WORKLOADS:
            print(f"--only: unknown workload {args.only}; one of {sorted(set(table) | set(WORKLOADS))}", file=sys.stderr)
            sys.exit(2)
        if args.only in table:
            r = table[args.only]()
        else:
            r, bufs = streamed(ctx, args.only, args.steps, args.warmup)
            del bufs
            r = rounded(r, 4)
        log(args.only, r)
        print(json.dumps({args.only: r}), flush=True)
        return

    main_name = "binary_512x2048"
    log("headline", main_name)
    head, (oset, x, y) = streamed(ctx, main_name, args.steps, args.warmup)
    log("headline", {k: (round(v, 4) if isinstance(v, float) else v) for k, v in head.items()})
    extra = {}
    rel = None
    if not args.only_main:
        _, _, hrows, hcols, _ = WORKLOADS[main_name]
        extra["headline_launch_distribution"] = launch_distribution(ctx, lambda: oset.gemv(x, hcols, y, hrows), 100)
        log("headline per-launch", extra["headline_launch_distribution"])
        rel = spot_check(ctx, oset, x, y)
        log("spot-check rel_l2", rel)
        del oset, x, y
        for name, fn in list(workloads.items()) + ([] if args.no_moe else list(moe_workloads.items())):
            extra[name] = fn()
            log(name, extra[name])
        ctrl = extra["stream_control_read_4gib"]["gbps"]
        extra["frac_of_stream_control"] = {name: round(r["gbps"] / ctrl, 4) for name, r in
                                           [(main_name, {"gbps": head["gbps"]})] + list(extra.items())
                                           if isinstance(r, dict) and "gbps" in r and name != "stream_control_read_4gib"}
    cpu = None if (args.no_cpu or args.only_main) else cpu_baseline()
    if cpu:
        log("cpu", cpu)
        extra["cpu_baselines"] = cpu_baselines()
        log("cpu baselines", extra["cpu_baselines"])

    traffic, tdet = (None, "not measured (--only-main or --no-traffic)")
    if not (args.only_main or args.no_traffic):
        log("traffic", "two rocprofv3 --pmc passes over the headline workload")
        traffic, tdet = live_traffic()
    if traffic is not None:
        extra["traffic_measurement"] = dict(tdet, source="rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes in this run",
                                            traffic_over_algorithmic=round(traffic / head["bytes"], 4))
    else:
        traffic = measured_traffic(main_name)
        extra["traffic_measurement"] = {"source": "committed profiles/gemv_binary_512x2048_streamed.pmc.json",
                                        "live_passes": tdet}
    log("traffic", traffic, extra["traffic_measurement"])
    line = {
        "metric": "packed-matvec GB/s (% HBM peak); MoE decode µs/token at batch 1",
        "value": round(head["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (counter-based N(0,0.02) weights packed on device, N(0,1) inputs)",
        "config": {"workload": f"config2 binary sign-plane organ 512x2048 (group 128, f16 mean|w|), "
                               f"{head['organs']} distinct organs streamed per launch, batch 1 per organ",
                   "organs_per_step": head["organs"], "bytes_per_step": head["bytes"],
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbps"], 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(head["gbps"] / HBM_PEAK_GBPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "parity_spot_check_rel_l2": rel,
        "extra": extra,
        "device": info["name"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
