"""Benchmark: the SiLVANN attention hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line.

Headline (`value`): config 2 of BASELINE.json — batched decode, 32 sequences with lengths U[1024, 32768]
from the seed, 32 q / 4 kv heads, head_dim 128, fp16 K/V in 256-position pages under seeded permuted page
tables — through the split-K decode door (silvann_gfx950_attention_decode_paged). A step is one decode of
the whole batch; `value` is its algorithmic bytes (each cached K and V row once, plus q, o and the page
table entries) × K over the K steps' own durations, inputs resident in HBM. Before each timed step a 1 GiB
buffer is written, so no step finds its inputs in the 256 MB Infinity Cache or the L2s; each step is bracketed
by hipEvents on the stream the library launches on, and the flushes fall outside them
(`wall_ms_per_step` in the lines is the wall clock of the whole timed region, flushes included).

`roofline` is the dominant kernel's (decode_split): algorithmic bytes ÷ its average launch duration, timed
live with hipEvents on the stream the library launches on, against 8 TB/s; `step_frac` is the same bytes over
the whole step (plan, split and merge launches and the gaps between them). `traffic` is the HBM bytes a launch
moves per rocprofv3 FETCH_SIZE + WRITE_SIZE, read from profiles/traffic.json when it holds a measurement of
this kernel and workload (else null).

`secondary` holds the other configurations' lines (decode GB/s for C1 and C5; prefill TFLOP/s for C3 and
C4 against 2.5 PFLOP/s dense fp16), each timed the same way.

With `--extra`, child processes (`--only 6`..`11`, each under a time limit, so a failure is recorded in its
entry and cannot take the headline down) add the fused TurboQuant residual (attention_residual_tq) over a 4-bit
and an 8-bit tier of C5's shape, in GB/s of codes, scales, q and residuals; the cache writer
(attention_cache_write_paged) placing C4's 2,048-row chunk, keys turned, in GB/s; GLM 5.3's latent attention
(64 heads over 131,072 512-wide latents, row 137 with k = v) in GB/s with its TFLOP/s beside; and C5 / C3
through the reference's own decode and rows verbs, whose door chains this library defers and runs fused. With
`--variants`, C2 once more with each of the split-K decode's opt-in forms, and C3 and C4 with each opt-in prefill
kernel (causal_duo, causal_pipe).

`cpu_baseline` is the reference's own x86_avx2 silicon family (oracle/_ref, built from the reference's
sources) over the same batch, its doors called through its nn table on the host cores — both of the
reference's decode routes (attention_scores + attention_mix; attention_weights + attention_residual_mix +
attention_finish), the faster reported. Pages are gathered to the reference's contiguous layout first,
outside the timing. Without oracle/_ref the C restatement (oracle/liboracle_attention.so, one core) is
timed instead, as "port".
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
METRIC = "decode-attn GB/s & % HBM peak; prefill-attn TFLOP/s & % MFMA peak"
KERNELS = ("decode_split", "decode_merge", "causal_mfma", "tq_split", "cache_write")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--variants", action="store_true",
                    help="also the decode's opt-in candidates (fused finish, transposing reads, inline plan, one "
                         "launch) and the prefill's (causal_duo, causal_pipe) as child-process lines")
    ap.add_argument("--extra", action="store_true",
                    help="also the lines of the section-f rows and the reference verbs (--only 6..11) as child processes")
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("BENCH_CPU_THREADS", "16")))
    ap.add_argument("--only", type=int, default=0,
                    help="time only this config (1-5: BASELINE.json's; 6, 7: a 4-bit / 8-bit TurboQuant tier; 8: the "
                         "cache writer on C4's chunk; 9: GLM 5.3's latent attention; 10, 11: C5 / C3 through the "
                         "reference's own decode / rows verb), no CPU leg")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run a plain 1 GiB device-to-device copy 5 times and exit: the known-size kernel the "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by")
    return ap.parse_args()


def prof_read(name):
    import silvann_amd
    L = silvann_amd.lib()
    ms, n = C.c_double(0), C.c_uint64(0)
    if L.silvann_gfx950_profile_read(name.encode(), C.byref(ms), C.byref(n)) != 0:
        raise RuntimeError("profile read failed")
    return ms.value, n.value


_FLUSH = {}


def _flush_l2():
    """Evict the caches between timed steps: write a 1 GiB buffer, four times the MI355X's 256 MB Infinity Cache
    (MALL) and far beyond its L2s, so every step reads its inputs from HBM."""
    import torch
    buf = _FLUSH.get("buf")
    if buf is None:
        buf = _FLUSH["buf"] = torch.empty(1 << 28, dtype=torch.int32, device="cuda:0")
    _FLUSH["n"] = _FLUSH.get("n", 0) + 1
    buf.fill_(_FLUSH["n"])


def time_steps(step, steps, warmup, kernel):
    """Warm up, then time exactly `steps` steps, each after a cache flush: the steps' own durations (hipEvents on
    torch's current stream, which the library is set to launch on, around each step, the flush outside them), the
    wall clock of the whole timed region between device synchronisations (flushes included), and the named
    kernel's average launch duration (the library's hipEvents around that kernel)."""
    import torch
    import silvann_amd
    L = silvann_amd.lib()
    stream = torch.cuda.current_stream()
    silvann_amd.doors.set_stream(stream)   # the library's launches, the flushes and the events on one stream
    for _ in range(warmup):
        _flush_l2()   # the flush buffer is allocated here, before any timing
        step()
    torch.cuda.synchronize()
    L.silvann_gfx950_profile_enable(1)
    for k in KERNELS:
        prof_read(k)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in evs:
        _flush_l2()
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    L.silvann_gfx950_profile_enable(0)
    step_s = sum(a.elapsed_time(b) for a, b in evs) * 1e-3
    kms, n = prof_read(kernel)
    others = {k: prof_read(k) for k in KERNELS if k != kernel}
    if silvann_amd.doors.launch_failed():
        raise RuntimeError("a launch failed during the timed steps")
    return {"step_s": step_s, "wall_s": wall}, kms / max(n, 1), others


def traffic_for(kernel, workload):
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text()).get(f"{kernel}:{workload}")
        # a measurement of an older build of the kernel is not this one's traffic
        return None if d is None or d.get("older_build") else d["traffic_bytes"]
    except Exception:
        return None


def decode_setup(w, dev):
    import torch
    from silvann_amd import verbs
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    lens = t(w.lens)
    pages = None if w.pages is None else t(w.pages)
    out = torch.zeros(w.rows * w.q_heads * w.head_dim, dtype=torch.float16, device=dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    need = verbs.decode_paged_scratch_bytes(w.q_heads, w.kv_heads, w.head_dim, w.most, w.rows)
    scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=dev)
    from silvann_amd import doors

    def step():
        doors.attention_decode_paged(out, w.q, w.k, w.v, pages, w.pages_row, w.page_size, w.k_row, lens, w.q_heads,
                                     w.kv_heads, w.head_dim, w.most, w.rows, scratch, over)
    return step, out, over


def causal_setup(w, dev):
    import torch
    from silvann_amd import doors
    pages = None if w.pages is None else torch.from_numpy(w.pages).to(dev)
    out = torch.zeros(w.rows * w.q_heads * w.head_dim, dtype=torch.float16, device=dev)
    over = torch.zeros(1, dtype=torch.int32, device=dev)

    def step():
        doors.attention_causal_paged(out, w.q, w.k, w.v, pages, w.page_size, w.q_heads, w.kv_heads, w.head_dim,
                                     w.first, w.rows, over)
    return step, out, over


def bench_decode(w, dev, steps, warmup):
    step, out, over = decode_setup(w, dev)
    tm, split_ms, others = time_steps(step, steps, warmup, "decode_split")
    b = w.io_bytes()
    merge_ms = others["decode_merge"][0] / max(others["decode_merge"][1], 1)
    return {
        "config": w.name, "unit": "GB/s", "value": b * steps / tm["step_s"] / 1e9,
        "ms_per_step": tm["step_s"] / steps * 1e3, "wall_ms_per_step": tm["wall_s"] / steps * 1e3,
        "bytes_per_step": b, "split_ms": split_ms, "merge_ms": merge_ms,
        "kernel_gbs": b / (split_ms * 1e-3) / 1e9, "frac": b / (split_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "step_frac": b * steps / tm["step_s"] / 1e9 / HBM_PEAK_GBS,
    }, out


def bench_causal(w, dev, steps, warmup):
    step, out, over = causal_setup(w, dev)
    tm, kms, _ = time_steps(step, steps, warmup, "causal_mfma")
    f = w.flops()
    return {
        "config": w.name, "unit": "TFLOP/s", "value": f * steps / tm["step_s"] / 1e12,
        "ms_per_step": tm["step_s"] / steps * 1e3, "wall_ms_per_step": tm["wall_s"] / steps * 1e3,
        "flops_per_step": f, "kernel_ms": kms, "kernel_tflops": f / (kms * 1e-3) / 1e12,
        "frac": f / (kms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS,
        "step_frac": f * steps / tm["step_s"] / 1e12 / FP16_PEAK_TFLOPS,
    }, out


def bench_tier(w, dev, steps, warmup):
    """The fused TurboQuant residual (attention_residual_tq) over one tier: GB/s of codes, scales, q and residuals."""
    import torch
    from silvann_amd import doors, verbs
    res = torch.zeros(w.rows * w.q_heads * (w.head_dim + 2), dtype=torch.float32, device=dev)
    scratch = torch.empty(max(verbs.residual_tq_scratch_bytes(w.q_heads, w.kv_heads, w.head_dim, w.length, w.d, w.rows), 4),
                          dtype=torch.uint8, device=dev)

    def step():
        doors.attention_residual_tq(res, w.q, w.k_codes, w.k_scales, w.v_codes, w.v_scales, w.q_heads, w.kv_heads,
                                    w.head_dim, w.length, w.d, w.rows, scratch)
    tm, kms, _ = time_steps(step, steps, warmup, "tq_split")
    ts = tm["step_s"]
    b = w.io_bytes()
    return {
        "config": w.name, "unit": "GB/s", "value": b * steps / ts / 1e9, "ms_per_step": wall / steps * 1e3,
        "bytes_per_step": b, "split_ms": kms, "kernel_gbs": b / (kms * 1e-3) / 1e9,
        "frac": b / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }, res


def bench_latent(w, dev, steps, warmup):
    """Latent attention (row 137, k = v): GB/s of latents read once, q and o, and the TFLOP/s of the two
    contractions (4·heads·latent_dim a position) beside it — the shape sits near the ridge of both rooflines."""
    step, out, over = decode_setup(w, dev)
    tm, split_ms, others = time_steps(step, steps, warmup, "decode_split")
    ts = tm["step_s"]
    pos = int(w.lens.astype("int64").sum())
    b = pos * w.head_dim * 2 + 2 * w.rows * w.q_heads * w.head_dim * 2
    f = 4 * w.q_heads * w.head_dim * pos
    merge_ms = others["decode_merge"][0] / max(others["decode_merge"][1], 1)
    return {
        "config": w.name, "unit": "GB/s", "value": b * steps / ts / 1e9, "ms_per_step": wall / steps * 1e3,
        "bytes_per_step": b, "flops_per_step": f, "split_ms": split_ms, "merge_ms": merge_ms,
        "kernel_gbs": b / (split_ms * 1e-3) / 1e9, "frac": b / (split_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernel_tflops": f / (split_ms * 1e-3) / 1e12,
    }, out


def bench_verb(n, dev, steps, warmup):
    """The reference's own verbs on this library's doors, no change to the caller: C5 through the decode verb
    (attention_scores then attention_mix, a deferred chain run as the split-K decode), or C3 through the rows verb
    (passes of causal_scores_grouped, causal_softmax, causal_mix, each run as the causal kernel). Wall-clock rate of
    whole steps; the kernel timing is the fused kernel's."""
    import torch
    from silvann_amd import verbs
    from silvann_amd import workloads as W
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    if n == 10:
        w = W.config5(dev=dev)
        L = int(w.lens[0])
        k, v = w.k, w.v
        scores = torch.empty(w.q_heads * L, dtype=torch.float32, device=dev)
        out = torch.empty(w.q_heads * w.head_dim, dtype=torch.float16, device=dev)

        def step():
            verbs.decode(w.q, k, v, scores, out, w.q_heads, w.kv_heads, w.head_dim, 0, L, over)
        kernel, units = "decode_split", w.io_bytes()
    else:
        w = W.config3(dev=dev)
        scores = torch.empty(256 * w.q_heads * w.rows, dtype=torch.float32, device=dev)
        out = torch.empty(w.rows * w.q_heads * w.head_dim, dtype=torch.float16, device=dev)

        def step():
            verbs.rows_attention(w.q, w.k, w.v, scores, out, w.q_heads, w.kv_heads, w.head_dim, w.first, w.rows, over)
        kernel, units = "causal_mfma", w.flops()
    tm, kms, _ = time_steps(step, steps, warmup, kernel)
    ts = tm["step_s"]
    if int(over.item()):
        raise RuntimeError(f"fault word {int(over.item()):#x}")
    per_step_kernel_ms = kms   # average launch; the rows verb launches one a pass
    if n == 10:
        return {"config": "C5 through the decode verb (scores -> mix)", "unit": "GB/s",
                "value": units * steps / ts / 1e9, "ms_per_step": wall / steps * 1e3, "bytes_per_step": units,
                "split_ms": per_step_kernel_ms}, out
    return {"config": "C3 through the rows verb (causal scores -> softmax -> mix, 256-row passes)", "unit": "TFLOP/s",
            "value": units * steps / ts / 1e12, "ms_per_step": wall / steps * 1e3, "flops_per_step": units,
            "kernel_ms_per_pass": per_step_kernel_ms}, out


def bench_write(w, dev, steps, warmup):
    """The cache writer (attention_cache_write_paged): a chunk's keys turned and its keys and values placed in
    their pages, GB/s of rows read and written and angles read."""
    import torch
    from silvann_amd import doors
    over = torch.zeros(1, dtype=torch.int32, device=dev)
    npr = w.pages.numel()

    def step():
        doors.attention_cache_write_paged(w.k_cache, w.v_cache, w.pages, npr, w.page_size, w.capacity, w.positions,
                                          w.rows, w.k, w.v, w.cs, w.rot, w.rows, w.kv_heads, w.head_dim, over)
    tm, kms, _ = time_steps(step, steps, warmup, "cache_write")
    ts = tm["step_s"]
    if int(over.item()):
        raise RuntimeError(f"cache writer fault word {int(over.item()):#x}")
    b = w.io_bytes()
    return {
        "config": w.name, "unit": "GB/s", "value": b * steps / ts / 1e9, "ms_per_step": wall / steps * 1e3,
        "bytes_per_step": b, "kernel_ms": kms, "kernel_gbs": b / (kms * 1e-3) / 1e9,
        "frac": b / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }, None


def isolated(n, steps, warmup, limit=240, env=None, variant=None):
    """`bench.py --only n` in a child process (with `env` added): the lines of kernels not yet measured on this
    hardware cannot take the headline down with them. Its JSON line, or what went wrong; `variant` names it."""
    import subprocess
    cmd = [sys.executable, str(Path(__file__).resolve()), "--only", str(n), "--steps", str(steps), "--warmup",
           str(warmup)]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=limit, env={**os.environ, **(env or {})})
    except subprocess.TimeoutExpired:
        return {"only": n, "variant": variant, "error": f"no answer within {limit} s"}
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"only": n, "variant": variant, "error": f"exit {r.returncode}: {r.stderr.strip()[-300:]}"}
    out = json.loads(lines[-1])
    if variant:
        out["variant"] = variant
    return out


def cpu_baseline(w, threads, budget=20.0):
    """The reference x86_avx2 family over the whole C2 batch (both decode routes, the faster reported); the C
    restatement on one core as "port" where oracle/_ref is absent."""
    import numpy as np
    from oracle.oracle import Oracle, RefFamily, ref_available
    q = w.q.cpu().numpy() if hasattr(w.q, "cpu") else w.q
    k = w.k.cpu().numpy() if hasattr(w.k, "cpu") else w.k
    v = w.v.cpu().numpy() if hasattr(w.v, "cpu") else w.v
    host = type(w)(**{**w.__dict__, "q": q, "k": k, "v": v})
    rows = [host.gathered(u) for u in range(w.rows)]
    qs = q.reshape(w.rows, -1)
    if ref_available():
        os.environ["SILVANN_CPU_THREADS"] = str(max(threads - 1, 0))
        R = RefFamily()
        routes = {"attention_scores+attention_mix": R.decode,
                  "attention_weights+attention_residual_mix+attention_finish": R.decode_tiered}
        kind, cores = "reference", threads
    else:
        O = Oracle()

        def port(qq, kk, vv, qh, kvh, hd, n):
            p = O.scores(qq, kk, qh, kvh, hd, n)
            return O.mix(p, vv, qh, kvh, hd, n)
        routes = {"oracle scores+mix": port}
        kind, cores = "port", 1
    best = None
    for name, fn in routes.items():
        reps, total, t_all = 0, 0.0, time.perf_counter()
        while True:
            for u in range(w.rows):
                kk, vv = rows[u]
                t0 = time.perf_counter()
                fn(qs[u], kk, vv, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
                total += time.perf_counter() - t0
            reps += 1
            if time.perf_counter() - t_all > budget / len(routes) or reps >= 400:
                break
        gbs = w.io_bytes() * reps / total / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, name, reps, total)
    gbs, name, reps, total = best
    return {"value": gbs, "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": f"full C2 batch ({w.rows} sequences, {int(w.lens.sum())} positions) x{reps}, route {name}, "
                      f"{total:.1f} s of CPU work; pages gathered to contiguous outside the timing"}


def cpu_baseline_prefill(w, threads, budget=10.0):
    """The reference x86_avx2 family's prefill doors beside the causal line: the last rows of the chunk (the heaviest,
    each over the whole prefix) through attention_causal_scores_grouped, attention_causal_softmax and
    attention_causal_mix, as the rows verb calls them (attention__abi.cuh:407-414), over the gathered contiguous cache,
    repeated for about `budget` seconds. TFLOP/s of unmasked (query, key) pairs, 4·q_heads·head_dim each."""
    import numpy as np
    from oracle.oracle import RefFamily, ref_available
    if not ref_available():
        return None
    host = lambda a: a.cpu().numpy() if hasattr(a, "cpu") else a  # noqa: E731
    qh, kvh, hd = w.q_heads, w.kv_heads, w.head_dim
    sample = 16
    first = w.first + w.rows - sample
    hw = type(w)(**{**w.__dict__, "q": host(w.q), "k": host(w.k), "v": host(w.v)})
    k, v = hw.gathered()
    q = hw.q[(w.rows - sample) * qh * hd:]
    os.environ["SILVANN_CPU_THREADS"] = str(max(threads - 1, 0))
    R = RefFamily()
    flops = 4 * qh * hd * sum(first + i + 1 for i in range(sample))
    reps, total = 0, 0.0
    while total < budget and reps < 100:
        t0 = time.perf_counter()
        p = R.causal_scores_grouped(q, k, qh, kvh, hd, first, sample)
        p = R.causal_softmax(p, qh, first, sample)
        R.causal_mix(p, v, qh, kvh, hd, first, sample)
        total += time.perf_counter() - t0
        reps += 1
    return {"value": flops * reps / total / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"the chunk's last {sample} rows (positions {first}..{first + sample - 1}, each over its whole "
                      f"prefix) x{reps}, causal_scores_grouped + causal_softmax + causal_mix, {total:.1f} s of CPU work; "
                      "pages gathered to contiguous outside the timing"}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported (every GPU box here has one "
              "GPU, and the attention path's sharding across GPUs is described, not built)", file=sys.stderr)
        sys.exit(2)
    import torch
    import silvann_amd
    from silvann_amd import workloads as W
    silvann_amd.lib()
    dev = torch.device("cuda:0")

    if a.copy_probe:
        src = torch.ones(1 << 29, dtype=torch.float16, device=dev)   # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 2, "launches": 5}), flush=True)
        return

    if a.only in (10, 11):
        r = bench_verb(a.only, dev, a.steps, a.warmup)[0]
        print(json.dumps(r), flush=True)
        return
    if a.only in W.LATENTS:
        r = bench_latent(W.LATENTS[a.only](dev=dev), dev, a.steps, a.warmup)[0]
        print(json.dumps(r), flush=True)
        return
    if a.only in W.WRITES:
        r = bench_write(W.WRITES[a.only](dev=dev), dev, a.steps, a.warmup)[0]
        print(json.dumps(r), flush=True)
        return
    if a.only in W.TIERS:
        r = bench_tier(W.TIERS[a.only](dev=dev), dev, a.steps, a.warmup)[0]
        print(json.dumps(r), flush=True)
        return
    if a.only:
        w = W.CONFIGS[a.only](dev=dev)
        r = (bench_decode if a.only in (1, 2, 5) else bench_causal)(w, dev, a.steps, a.warmup)[0]
        print(json.dumps(r), flush=True)
        return

    w2 = W.config2(dev=dev)
    head, _ = bench_decode(w2, dev, a.steps, a.warmup)
    secondary = []
    if not a.no_secondary:
        for n in (5, 1):
            w = W.CONFIGS[n](dev=dev)
            secondary.append(bench_decode(w, dev, max(5, a.steps // 2), a.warmup)[0])
            del w
        for n in (3, 4):
            w = W.CONFIGS[n](dev=dev)
            line = bench_causal(w, dev, max(3, a.steps // 4), min(a.warmup, 2))[0]
            if n == 4 and not a.no_cpu:
                line["cpu_baseline"] = cpu_baseline_prefill(w, a.cpu_threads)
            secondary.append(line)
            del w
        torch.cuda.empty_cache()
        if a.extra:
            for n in sorted([*W.TIERS, *W.WRITES, *W.LATENTS]):
                secondary.append(isolated(n, max(5, a.steps // 2), a.warmup))
        if a.variants:
            secondary.append(isolated(2, a.steps, a.warmup, env={"SILVANN_GFX950_DECODE_FUSED": "1"},
                                      variant="fused finish (no merge launch)"))
            secondary.append(isolated(2, a.steps, a.warmup, env={"SILVANN_GFX950_DECODE_VTR": "1"},
                                      variant="transposing V^T reads"))
            secondary.append(isolated(2, a.steps, a.warmup, env={"SILVANN_GFX950_DECODE_INLINE": "1"},
                                      variant="plan inside decode_split (no plan launch)"))
            secondary.append(isolated(2, a.steps, a.warmup,
                                      env={"SILVANN_GFX950_DECODE_INLINE": "1", "SILVANN_GFX950_DECODE_FUSED": "1"},
                                      variant="one launch a step (inline plan + fused finish)"))
            secondary.append(isolated(9, max(5, a.steps // 2), a.warmup, env={"SILVANN_GFX950_DECODE_LATENT": "wide"},
                                      variant="latent attention, four head blocks a workgroup (decode_latent)"))
            for kernel, what in (("duo", "causal_duo: two waves a SIMD over alternate key tiles"),
                                 ("pipe", "causal_pipe: one wave a SIMD, pipelined two tiles deep")):
                for n in (3, 4):
                    secondary.append(isolated(n, max(3, a.steps // 4), min(a.warmup, 2),
                                              env={"SILVANN_GFX950_PREFILL": kernel}, variant=what))
            for n in (1, 5):   # the launch-bound and the longest decode in one launch
                secondary.append(isolated(n, max(5, a.steps // 2), a.warmup,
                                          env={"SILVANN_GFX950_DECODE_INLINE": "1", "SILVANN_GFX950_DECODE_FUSED": "1"},
                                          variant="one launch a step (inline plan + fused finish)"))
        if a.extra:
            for n in (10, 11):
                secondary.append(isolated(n, max(5, a.steps // 2), a.warmup))
    cpu = None if a.no_cpu else cpu_baseline(w2, a.cpu_threads)

    line = {
        "metric": METRIC,
        "value": round(head["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic: seeded N(0,1) fp16 q/k/v, seeded lengths and permuted page tables",
        "config": {"workload": w2.name, "sequences": w2.rows, "positions": int(w2.lens.sum()),
                   "q_heads": w2.q_heads, "kv_heads": w2.kv_heads, "head_dim": w2.head_dim,
                   "page_size": w2.page_size, "bytes_per_step": head["bytes_per_step"]},
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["frac"], 4), "step_frac": round(head["step_frac"], 4),
                     "traffic": traffic_for("decode_split", w2.name),
                     "kernel": "decode_split", "kernel_ms": round(head["split_ms"], 5),
                     "merge_ms": round(head["merge_ms"], 5)},
        "secondary": [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in s.items()} for s in secondary],
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
