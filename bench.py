"""Benchmark of the MI355X attention hot path.

Headline (one JSON line): config 2 of the north star -- LLaMA-2-style GQA causal
prefill, f32, B=4, Hq=32, Hkv=8, T=2048, d=128, Q/K/V ~ N(0,1) with a per-
position scale U[0.5, 1.5] on Q and K (seeded, synthetic).  A step is one
prefill forward over the whole batch with inputs resident in HBM; value is
attention TFLOP/s (2 FLOP per multiply-add of QK^T and PV over the T(T+1)/2
unmasked pairs per head).  Before the W warm-up steps the prefill runs untimed
for ~60 ms (clock_settle_ms) so the GPU has left its idle clock state.  The
same line carries:
  * roofline -- the prefill kernel's average launch time from HIP events on
    the launch stream, against MI355X's fp32 matrix peak (157.3 TFLOP/s);
  * decode   -- config 3: 64 single-token decode steps (append + attend) over
    a ragged KV cache, B=32, Hq=32, Hkv=8, d=128, L0 ~ U[512, 4096], as KV-read
    GB/s against HBM peak (8 TB/s);
  * cpu_baseline -- the reference's own CPU path for GQA attention restated in
    C (oracle/rayon_path.c, a "port": its AVX2/FMA GEMM and GEMV kernels, Rayon
    splits, repeat-KV, mask, softmax; Tensor::cat of the cache for decode),
    timed on this host's cores on a bounded sample of the same workload, with
    as many threads as Rayon's global pool would take here (the available
    parallelism: affinity mask and cgroup quota).  The flash legs (configs 1,
    4, 5a) time the oracle's flash_attention_forward, which is scalar like the
    reference's;
  * other_configs -- configs 1, 4, 5a and 5b, a head-dim-256 causal prefill,
    the G = 8 decode and the decode layer steps, each with its own kernel
    time, roofline fraction and cpu_baseline.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--headline]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

PEAK_FP32_MATRIX_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on
# the `--probe` workload, each scaled by its reading for a plain 1 GiB device copy
# (FETCH_SIZE x2.00, WRITE_SIZE x1.00).  Config 2 prefill: 224.4 MB read + 134.2 MB
# written (algorithmic 201.3 + 134.2; part of the shared K/V is fetched into two
# XCDs' L2).  Config 3 decode step (one launch, split heads merged inside it):
# 646.0 MB read + 1.8 MB written (algorithmic 645.0 + 0.8, plus the partial records
# of split heads).  Config 5b: 123.4 + 0.33 (algorithmic 123.2 + 0.33).  Config-3
# decode prologue: 109.2 + 4.7 (algorithmic 101.2 + 0.8; partial tiles and x per
# XCD).  GPT-2 decode attend: 104.4 + 0.3 (algorithmic 104.2 + 0.3).  Config 1:
# 1.1 + 0.26 (algorithmic 0.79 + 0.26).  Config 4: 272.2 + 67.1 (algorithmic
# 201.3 + 67.1; the persistent workgroups of a KV head on one XCD re-fetch part of
# its 8.4 MB of K/V, more than the XCD's 4 MB L2).  Config 5a: 187.0 + 61.4
# (algorithmic 184.3 + 61.4).  G = 8 decode step: 677.2 + 3.25 (algorithmic
# 681.3 + 1.3, plus the 16-row partial records of split heads).  d = 256 causal
# prefill (B = 1, H = 16, T = 4096): 260.3 + 67.8 (algorithmic 201.3 + 67.1).  d = 512
# causal prefill (deep kernel, same shape): 1585.6 + 134.2 (algorithmic 402.7 + 134.2;
# the units of a KV head re-fetch its 16.8 MB of K/V, more than the XCD's 4 MB L2).
TRAFFIC_PREFILL_CONFIG2 = round(224.4e6 + 134.2e6)
TRAFFIC_DECODE_CONFIG3_STEP = round(646.0e6 + 1.8e6)
TRAFFIC_CROSS_CONFIG5B = round(123.4e6 + 0.33e6)
TRAFFIC_PROLOGUE_CONFIG3 = round(109.2e6 + 4.7e6)
TRAFFIC_ATTEND_GPT2 = round(104.4e6 + 0.3e6)
TRAFFIC_PREFILL_CONFIG1 = round(1.1e6 + 0.26e6)
TRAFFIC_PREFILL_CONFIG4 = round(272.2e6 + 67.1e6)
TRAFFIC_PREFILL_CONFIG5A = round(187.0e6 + 61.4e6)
TRAFFIC_DECODE_G8_STEP = round(677.2e6 + 3.25e6)
TRAFFIC_PREFILL_D256 = round(260.3e6 + 67.8e6)
TRAFFIC_PREFILL_D512 = round(1585.6e6 + 134.2e6)


def cpu_threads():
    """Threads of the CPU legs: the parallelism Rayon's global pool takes by
    default (std::thread::available_parallelism on Linux: the CPUs of the
    scheduler affinity mask, capped by a cgroup v2 cpu.max quota)."""
    n = len(os.sched_getaffinity(0))
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return max(1, n)


def host_cpu():
    """The host facts each cpu_baseline records."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


def with_host(rec):
    rec.update(host_cpu())
    return rec


def load_pkg():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import nne_testlib
    return nne_testlib.load_package()


def causal_flops(b, hq, t, d):
    return 4.0 * b * hq * d * t * (t + 1) / 2.0


def full_flops(b, hq, tq, tk, d):
    return 4.0 * b * hq * d * tq * tk


def config2_inputs(torch, dev, b=4, hq=32, hkv=8, t=2048, d=128, seed=0x5EED0002):
    g = torch.Generator(device=dev).manual_seed(seed)
    s = torch.rand(t, generator=g, device=dev) + 0.5
    q = torch.randn(b, hq, t, d, generator=g, device=dev) * s[None, None, :, None]
    k = torch.randn(b, hkv, t, d, generator=g, device=dev) * s[None, None, :, None]
    v = torch.randn(b, hkv, t, d, generator=g, device=dev)
    return q, k, v


def gpu_ms_per_call(torch, call, reps, queued):
    """Device time per call over reps back-to-back calls (HIP events on the
    current stream).  queued: a bounded spin kernel (torch.cuda._sleep) holds
    the stream while Python issues the calls, so the figure is the GPU's own
    rate rather than the Python issue rate."""
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    if queued:
        torch.cuda._sleep(int(2e5) * reps)
    e0.record(stream)
    for i in range(reps):
        call(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def settle_clocks(torch, call, target_ms=60.0):
    """Runs call() back to back for about target_ms of wall time.  A GPU
    coming out of idle raises its clocks over its first ~30 ms of work: on
    MI355X the config-2 prefill takes 1.30 ms on the first launches and 1.07 ms
    from the 25th on.  Returns the time spent."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < target_ms:
        for _ in range(4):
            call()
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def time_prefill(nne, torch, q, k, v, causal, steps, warmup, out, q_offset=0):
    for _ in range(warmup):
        nne.attention_forward(q, k, v, causal, q_offset=q_offset, out=out)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        nne.attention_forward(q, k, v, causal, q_offset=q_offset, out=out)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = ev0.elapsed_time(ev1) / steps
    return wall * 1e3 / steps, kernel_ms


def bench_decode(nne, torch, dev, steps=64, warmup=4, seed=0x5EED0003, hq=32, hkv=8,
                 workload="config3: decode B=32 Hq=32 Hkv=8 d=128 "
                          "L0~U[512,4096] ragged, 64 steps append+attend, f32",
                 traffic=None):
    """Config 3: B=32, Hq=32, Hkv=8, d=128, ragged lengths, 64 append+attend
    steps.  hq/hkv give other group sizes on the same lengths (Hq=64, Hkv=8 is
    LLaMA-2-70B's grouping: 8 query rows per KV head)."""
    import numpy as np
    b, d = 32, 128
    rng = np.random.default_rng(seed)
    lens0 = rng.integers(512, 4097, size=b).astype(np.int32)
    cap = 4096 + steps + warmup
    cache = nne.KVCache(1, b, hkv, cap, d, device=dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    cache.k[0].normal_(generator=g)
    cache.v[0].normal_(generator=g)
    qs = torch.randn(steps, b, hq, 1, d, generator=g, device=dev)
    kn = torch.randn(steps, b, hkv, 1, d, generator=g, device=dev)
    vn = torch.randn(steps, b, hkv, 1, d, generator=g, device=dev)
    out = torch.empty(b, hq, 1, d, device=dev)
    cache.set_lengths(0, lens0)
    for i in range(warmup):
        cache.decode_step(0, qs[i], kn[i], vn[i], out=out)
    step = lambda i: cache.decode_step(0, qs[i], kn[i], vn[i], out=out)
    cache.set_lengths(0, lens0)
    ms = gpu_ms_per_call(torch, step, steps, queued=True) * steps
    cache.set_lengths(0, lens0)
    ms_host = gpu_ms_per_call(torch, step, steps, queued=False) * steps
    # K+V rows read once per KV head (GQA-shared) after each step's append,
    # plus q/o and the appended rows.
    total = 0.0
    for i in range(steps):
        total += float((lens0 + i + 1).sum()) * hkv * d * 4 * 2
        total += 2 * b * hq * d * 4 + b * hkv * d * 4 * 2
    gbs = total / (ms / 1e3) / 1e9
    return {"metric": "decode KV-read GB/s", "value": round(gbs, 1), "unit": "GB/s",
            "steps": steps, "ms_per_step": round(ms / steps, 4),
            "host_paced_ms_per_step": round(ms_host / steps, 4),
            "bytes_per_step": round(total / steps),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic},
            "config": {"workload": workload}}


RP_RESTATES = ("gemm_2d_a_bt_avx2_fma_parallel / gemv_a_bt_m1_avx2_fma_parallel (QK^T) and "
               "gemm_2d_avx2_fma_parallel / gemv_m1_avx2_fma (PV) under the batched matmul "
               "drivers, matmul.rs:30-80, 87-560, 749-1056, 1112-1318; softmax fast path with "
               "find_row_max_avx2 / scale_row_avx2, reduce.rs:234-330; repeat-KV as Storage::zeros "
               "+ broadcast add, llama.rs:256-266, ops.rs:43-84; the -1e4 mask as a broadcast add, "
               "llama.rs:277-292; to_contiguous gathers, mod.rs:184-197")


def _rp():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import nne_testlib as T
    return T


def _components(times, digits=4):
    return {k: round(v, digits) for k, v in times.items() if v > 0}


def cpu_baseline(reps=2):
    """Config 2 in full on the reference's own CPU path for GQA attention
    (llama.rs:253-296 through its AVX2/FMA GEMMs, oracle/rayon_path.c), median
    of reps calls."""
    import numpy as np
    T = _rp()
    threads = cpu_threads()
    b, hq, hkv, t, d = 4, 32, 8, 2048, 128
    rng = np.random.default_rng(0x5EED0002)
    s = rng.uniform(0.5, 1.5, size=t).astype(np.float32)
    q = rng.standard_normal((b, hq, t, d), dtype=np.float32) * s[None, None, :, None]
    k = rng.standard_normal((b, hkv, t, d), dtype=np.float32) * s[None, None, :, None]
    v = rng.standard_normal((b, hkv, t, d), dtype=np.float32)
    runs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        _, comp = T.rp_attention(q, k, v, mode="gqa", causal=True, threads=threads)
        runs.append((time.perf_counter() - t0, comp))
    el, comp = sorted(runs, key=lambda r: r[0])[len(runs) // 2]
    flops = causal_flops(b, hq, t, d)
    return with_host({
        "value": round(flops / el / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
        "kind": "port", "restates": RP_RESTATES,
        "sample": "config 2 in full (B=4, Hq=32, Hkv=8, T=2048, d=128, causal), "
                  "GroupedQueryAttention::forward_gqa_cached steps 4-7 (llama.rs:253-296) on the "
                  "reference's CPU path: repeat-KV, QK^T, scale, -1e4 mask, softmax, PV (f32, "
                  "AVX2/FMA, %d threads), median of %d: %.2f s; FLOPs counted like the GPU "
                  "(unmasked pairs only)" % (threads, reps, el),
        "components_s": _components(comp)})


def flash_cpu_baseline(b, h, t, d, causal, std, sample, reps=1, seed=0x5EED0004):
    """Oracle flash_attention_forward (flash_attention.rs:19-199, br = bc = 64
    as in the FlashAttention layer) on the host cores, parallel over the B*H
    heads as the reference is (:69); median of reps calls."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import nne_testlib as T
    threads = cpu_threads()
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((b, h, t, d), dtype=np.float32) * std for _ in range(3))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        T.ref_flash(q, k, v, causal, br=64, bc=64, threads=threads)
        times.append(time.perf_counter() - t0)
    el = sorted(times)[len(times) // 2]
    fl = causal_flops(b, h, t, d) if causal else full_flops(b, h, t, t, d)
    return with_host({
        "value": round(fl / el / 1e12, 6), "unit": "TFLOP/s", "cores": min(threads, b * h),
        "kind": "port",
        "sample": "%s; flash_attention_forward restated from flash_attention.rs:19-199 "
                  "(br = bc = 64, f32), parallel over the B*H heads as the reference's "
                  "par_chunks_mut (:69) on a pool of %d threads, %s, median of %d: %.3f s" % (
                      sample, threads, "causal" if causal else "non-causal", reps, el)})


def cross_cpu_baseline(b=8, h=20, tq=8, tk=1500, d=64, reps=3, seed=0x5EED0005):
    """Config 5b in full on the reference's CPU path for cross-attention
    (attention.rs:193-203): q and the slot's K/V are the transposed views of
    their [B, T, H, d] projections, so matmul_transposed_b and matmul gather
    them (to_contiguous) before the AVX2 kernels."""
    import numpy as np
    T = _rp()
    threads = cpu_threads()
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, tq, h, d), dtype=np.float32)
    k, v = (rng.standard_normal((b, tk, h, d), dtype=np.float32) for _ in range(2))
    runs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        _, comp = T.rp_attention(q, k, v, mode="cross", q_bthd=True, kv_bthd=True,
                                 threads=threads)
        runs.append((time.perf_counter() - t0, comp))
    el, comp = sorted(runs, key=lambda r: r[0])[len(runs) // 2]
    by = (2 * b * h * tk * d + 2 * b * h * tq * d) * 4
    return with_host({
        "value": round(by / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "restates": RP_RESTATES,
        "sample": "config 5b in full (B=8, H=20, 8 queries onto 1500 frames, d=64): "
                  "forward_cross_attention_cached steps 3-5 (attention.rs:193-203) on the "
                  "reference's CPU path, q/K/V as the transposed views the projections leave "
                  "(gathered by to_contiguous), scale as a broadcast mul, %d threads, median of "
                  "%d: %.3f s; bytes counted like the GPU line" % (threads, reps, el),
        "components_s": _components(comp)})


def decode_cpu_baseline(seed=0x5EED0003, n_seq=8, steps=4, shape=(32, 32, 8, 128),
                        len_range=(512, 4096), label="config 3 decode step", mode="gqa"):
    """Decode steps (t = 1, append then attend) on the reference's CPU path:
    a ragged batch needs one B = 1 call per sequence (its slots hold one
    length), each Tensor::cat-ing its K and V slot (ops.rs:215-275) and then
    attending (llama.rs:239-296 for "gqa", attention.rs:79-122 for "mha").
    The first n_seq sequences of the workload for `steps` steps."""
    import numpy as np
    T = _rp()
    threads = cpu_threads()
    b, hq, hkv, d = shape
    rng = np.random.default_rng(seed)
    lens = rng.integers(len_range[0], len_range[1] + 1, size=b).astype(np.int32)[:n_seq].copy()
    cap = int(lens.max()) + steps
    kc = rng.standard_normal((n_seq, hkv, cap, d), dtype=np.float32)
    vc = rng.standard_normal((n_seq, hkv, cap, d), dtype=np.float32)
    qs = rng.standard_normal((steps, n_seq, hq, d), dtype=np.float32)
    kns = rng.standard_normal((steps, n_seq, hkv, d), dtype=np.float32)
    vns = rng.standard_normal((steps, n_seq, hkv, d), dtype=np.float32)
    t0 = time.perf_counter()
    _, comp = T.rp_decode_run(qs, kc, vc, lens, kns, vns, mode=mode, threads=threads)
    el = time.perf_counter() - t0
    total = 0.0
    for i in range(steps):
        total += float((lens + i + 1).sum()) * hkv * d * 4 * 2 + 2 * n_seq * hq * d * 4 \
            + n_seq * hkv * d * 8
    cat_s = comp.get("cat", 0.0)
    return with_host({
        "value": round(total / el / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
        "restates": "Tensor::cat, ops.rs:215-275 (serial, per element); " + RP_RESTATES,
        "sample": "%s (B=%d, Hq=%d, Hkv=%d, d=%d): the first %d sequences (lengths %d-%d) for %d "
                  "steps, one B = 1 call per sequence as the reference must for ragged lengths: "
                  "Tensor::cat of the K and V slots, then %s on the reference's CPU path (%d "
                  "threads): %.2f s, of which the cat copies %.2f s; bytes counted like the GPU "
                  "line" % (label, b, hq, hkv, d, n_seq, int(lens.min()), int(lens.max()), steps,
                            "repeat-KV, QK^T, scale, softmax, PV" if hq > hkv else
                            "QK^T, scale, softmax, PV", threads, el, cat_s),
        "value_without_cat": round(total / max(el - cat_s, 1e-9) / 1e9, 4),
        "components_s": _components(comp)})


def prologue_cpu_baseline(seed=0x5EED0014, reps=15):
    """One config-3 decode prologue step (B = 32 rows) on the reference's CPU
    path: per sequence (one B = 1 call each) the q/k/v Linear layers
    (linear.rs:47-57: a GEMV, gemv_a_bt_m1_avx2_fma_parallel, per projection)
    and RotaryEmbedding::apply on q and k (llama.rs:109-157).  Median of reps
    steps."""
    import numpy as np
    T = _rp()
    threads = cpu_threads()
    b, hq, hkv, d = 32, 32, 8, 128
    c = hq * d
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, c), dtype=np.float32)
    w = [rng.standard_normal((h * d, c), dtype=np.float32) * (1.0 / c) ** 0.5 for h in (hq, hkv, hkv)]
    cos, sin = T.ref_rope_tables(4200, d)
    pos = rng.integers(512, 4097, size=b).astype(np.int32)
    runs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        _, _, _, comp = T.rp_qkv_rope_run(x, *w, None, None, None, cos, sin, pos, hq, hkv,
                                          threads=threads)
        runs.append((time.perf_counter() - t0, comp))
    el, comp = sorted(runs, key=lambda r: r[0])[len(runs) // 2]
    pbytes = (hq + 2 * hkv) * d * c * 4 + b * c * 4 + b * (hq + 2 * hkv) * d * 4
    return with_host({
        "value": round(pbytes / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "restates": "Linear::forward, linear.rs:47-57, via matmul_transposed_b -> "
                    "gemv_a_bt_m1_avx2_fma_parallel (matmul.rs:888-1056); "
                    "RotaryEmbedding::apply, llama.rs:109-157 (neg, cat, broadcast mul, add)",
        "sample": "one config-3 decode prologue step in full (32 rows, d_model 4096, Hq=32, "
                  "Hkv=8, d=128), one B = 1 call per sequence as the reference runs a ragged "
                  "batch (each row streams the 100.7 MB of weights again), %d threads, median of "
                  "%d steps: %.4f s; bytes per step counted like the GPU line" % (threads, reps, el),
        "components_s": _components(comp, 5)})


def bench_decode_layer(nne, torch, dev, steps=32, seed=0x5EED0013):
    """Config 3 as a GQA decode layer step (llama.rs:205-300, t = 1) minus
    the output GEMM: the fused projection + RoPE launch on packed weights
    (d_model 4096 = Hq * d), then the append + attend launch.  Three layers'
    weights (3 x 100.7 MB) rotate so no step finds its weights in the 256 MB
    MALL, as in a model whose layers run in turn."""
    import numpy as np
    b, hq, hkv, d = 32, 32, 8, 128
    c = hq * d
    rng = np.random.default_rng(seed)
    lens0 = rng.integers(512, 4097, size=b).astype(np.int32)
    cap = 4096 + 2 * steps + 8
    g = torch.Generator(device=dev).manual_seed(seed)
    bound = (1.0 / c) ** 0.5
    packed = []
    for _ in range(3):
        w = [(torch.rand(n * d, c, generator=g, device=dev) * 2 - 1) * bound
             for n in (hq, hkv, hkv)]
        packed.append(nne.qkv_pack(w[0], w[1], w[2], hq, hkv))
        del w
    rope = nne.RotaryEmbedding(d, cap, device=dev)
    cache = nne.KVCache(1, b, hkv, cap, d, device=dev)
    cache.k[0].normal_(generator=g)
    cache.v[0].normal_(generator=g)
    xs = torch.randn(steps, b, c, generator=g, device=dev)
    q = torch.empty(b, hq, 1, d, device=dev)
    kn = torch.empty(b, hkv, 1, d, device=dev)
    vn = torch.empty(b, hkv, 1, d, device=dev)
    out = torch.empty(b, hq, 1, d, device=dev)
    cache.set_lengths(0, lens0)
    lens_dev = cache.lens_dev[0]
    lens_host = cache.lens_host[0]

    def prologue(i):
        nne.qkv_rope(xs[i % steps], packed[i % 3], None, None, None, rope, lens_dev, lens_host,
                     hq, hkv, q, kn, vn)

    def layer_step(i):
        prologue(i)
        cache.decode_step(0, q, kn, vn, out=out)

    for i in range(3):
        prologue(i)
    pro_ms = gpu_ms_per_call(torch, prologue, steps, queued=True)
    layer_step(0)
    cache.set_lengths(0, lens0)
    step_ms = gpu_ms_per_call(torch, layer_step, steps, queued=True)
    wbytes = (hq + 2 * hkv) * d * c * 4
    pbytes = wbytes + b * c * 4 + b * (hq + 2 * hkv) * d * 4
    gbs = pbytes / (pro_ms / 1e3) / 1e9
    flops = 2.0 * b * c * (hq + 2 * hkv) * d
    return {"workload": "config3 decode layer step: fused q/k/v projection + RoPE (d_model "
                        "4096, packed weights, 3 layers rotated) + append/attend",
            "prologue_ms": round(pro_ms, 4), "prologue_GB/s": round(gbs, 1),
            "prologue_TFLOP/s": round(flops / (pro_ms / 1e3) / 1e12, 2),
            "prologue_frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "prologue_bytes": pbytes, "layer_step_ms": round(step_ms, 4),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "kernel": "qkv_rope_kernel", "bytes": pbytes,
                         "traffic": TRAFFIC_PROLOGUE_CONFIG3}}


def bench_mha_decode_layer(nne, torch, dev, steps=32, layers=12, seed=0x5EED0015):
    """GPT-2-small-style MultiHeadAttention decode step (attention.rs:51-129
    with t = 1; d_model 768, 12 heads, d = 64) for B = 32 sequences with
    cached lengths U[128, 1024]: the fused biased q/k/v projection (no RoPE)
    on packed weights, then the append + attend launch; the output GEMM is
    left out.  The q/k/v weights of 12 layers rotate, as in the model, and
    so do 3 layers' KV caches (3 x 217 MB at capacity, past the 256 MB MALL;
    with one cache re-read every step, loads that allocate in the MALL would
    find it there, which a 12-layer model never does)."""
    import numpy as np
    b, h, d = 32, 12, 64
    c = h * d
    rng = np.random.default_rng(seed)
    lens0 = rng.integers(128, 1025, size=b).astype(np.int32)
    cap = 1024 + 2 * steps + 8
    g = torch.Generator(device=dev).manual_seed(seed)
    bound = (1.0 / c) ** 0.5
    packed, biases = [], []
    for _ in range(layers):
        w = [(torch.rand(c, c, generator=g, device=dev) * 2 - 1) * bound for _ in range(3)]
        packed.append(nne.qkv_pack(w[0], w[1], w[2], h, h))
        biases.append([(torch.rand(c, generator=g, device=dev) * 2 - 1) * bound for _ in range(3)])
        del w
    n_kv = 3
    cache = nne.KVCache(n_kv, b, h, cap, d, device=dev)
    for layer in range(n_kv):
        cache.k[layer].normal_(generator=g)
        cache.v[layer].normal_(generator=g)
    xs = torch.randn(steps, b, c, generator=g, device=dev)
    q = torch.empty(b, h, 1, d, device=dev)
    kn = torch.empty(b, h, 1, d, device=dev)
    vn = torch.empty(b, h, 1, d, device=dev)
    out = torch.empty(b, h, 1, d, device=dev)

    def reset():
        for layer in range(n_kv):
            cache.set_lengths(layer, lens0)

    reset()

    def prologue(i):
        bq, bk, bv = biases[i % layers]
        nne.qkv_rope(xs[i % steps], packed[i % layers], bq, bk, bv, None, None, None, h, h, q, kn,
                     vn, head_dim=d)

    def attend(i):
        cache.decode_step(i % n_kv, q, kn, vn, out=out)

    def layer_step(i):
        prologue(i)
        attend(i)

    for i in range(3):
        prologue(i)
    pro_ms = gpu_ms_per_call(torch, prologue, steps, queued=True)
    reset()
    att_ms = gpu_ms_per_call(torch, attend, steps, queued=True)
    reset()
    step_ms = gpu_ms_per_call(torch, layer_step, steps, queued=True)
    kv_bytes = 0.0
    for i in range(steps):   # step i appends to layer i % n_kv, its (i // n_kv + 1)-th row
        kv_bytes += float((lens0 + i // n_kv + 1).sum()) * h * d * 4 * 2 + 2 * b * h * d * 4 + b * h * d * 8
    kv_bytes /= steps
    pbytes = 3 * c * c * 4 + 3 * c * 4 + b * c * 4 + 3 * b * c * 4
    return {"workload": "GPT-2-small MHA decode layer step (d_model 768, 12 heads, d 64, B=32, "
                        "L0~U[128,1024]): fused biased q/k/v projection (12 layers' weights "
                        "rotated) + append/attend (3 layers' KV caches rotated)",
            "prologue_ms": round(pro_ms, 4),
            "prologue_GB/s": round(pbytes / (pro_ms / 1e3) / 1e9, 1),
            "attend_ms": round(att_ms, 4),
            "attend_GB/s": round(kv_bytes / (att_ms / 1e3) / 1e9, 1),
            "attend_frac_hbm": round(kv_bytes / (att_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
            "layer_step_ms": round(step_ms, 4),
            "roofline": {"bound": "hbm", "achieved": round(kv_bytes / (att_ms / 1e3) / 1e9, 1),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(kv_bytes / (att_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                         "kernel": "splitk_kernel (append + attend)", "bytes": round(kv_bytes),
                         "traffic": TRAFFIC_ATTEND_GPT2}}


def probe(nne, torch, dev):
    """Fixed, short workload for rocprofv3 --pmc runs (one counter set per run)."""
    x = torch.empty(1 << 28, dtype=torch.float32, device=dev)     # 1 GiB
    x.fill_(1.0)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    q, k, v = config2_inputs(torch, dev)
    out = torch.empty_like(q)
    for _ in range(3):
        nne.attention_forward(q, k, v, True, out=out)
    torch.cuda.synchronize()
    del q, k, v, out
    bench_decode(nne, torch, dev, steps=8, warmup=1)
    torch.cuda.synchronize()
    g = torch.Generator(device=dev).manual_seed(0x5EED0005)
    qx = torch.randn(8, 20, 8, 64, generator=g, device=dev)
    ox = torch.empty_like(qx)
    kvs = [(torch.randn(8, 20, 1500, 64, generator=g, device=dev),
            torch.randn(8, 20, 1500, 64, generator=g, device=dev)) for _ in range(3)]
    for i in range(6):                        # config 5b, K/V sets rotated past the MALL
        nne.attention_forward(qx, kvs[i % 3][0], kvs[i % 3][1], False, out=ox)
    torch.cuda.synchronize()
    bench_decode_layer(nne, torch, dev, steps=6)
    torch.cuda.synchronize()
    bench_mha_decode_layer(nne, torch, dev, steps=6)
    torch.cuda.synchronize()
    q1, k1, v1 = (torch.randn(1, 4, 256, 64, generator=g, device=dev) for _ in range(3))
    o1 = torch.empty_like(q1)
    for _ in range(6):                        # config 1
        nne.attention_forward(q1, k1, v1, True, out=o1)
    torch.cuda.synchronize()
    del q1, k1, v1, o1
    for (bb, h, tt, dd, causal, std, calls) in ((1, 16, 16384, 64, True, 0.5, 2),   # config 4
                                                (8, 20, 1500, 64, False, 1.0, 3),   # config 5a
                                                (1, 16, 4096, 256, True, 1.0, 3),   # d = 256
                                                (1, 16, 4096, 512, True, 1.0, 3)):  # d = 512
        q, k, v = (torch.randn(bb, h, tt, dd, generator=g, device=dev) * std for _ in range(3))
        o = torch.empty_like(q)
        for _ in range(calls):
            nne.attention_forward(q, k, v, causal, out=o)
        torch.cuda.synchronize()
        del q, k, v, o
    bench_decode(nne, torch, dev, steps=8, warmup=1, hq=64, seed=0x5EED0016)   # G = 8 decode
    torch.cuda.synchronize()
    print("probe done", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--all", action="store_true",
                    help="kept for old command lines: every config is measured by default")
    ap.add_argument("--headline", action="store_true",
                    help="measure only the config-2 prefill and the config-3 decode")
    ap.add_argument("--probe", action="store_true",
                    help="counter-collection run: a 1 GiB device copy (calibrates FETCH_SIZE/"
                         "WRITE_SIZE), 3 config-2 prefills, 8 config-3 decode steps, 6 "
                         "config-5b cross-attention calls, 6 config-3 and 6 GPT-2 decode layer "
                         "steps, 6 config-1 prefills, 2 config-4, 3 config-5a, 3 d=256 and 3 "
                         "d=512 prefills, 8 G=8 decode steps")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    nne = load_pkg()
    nne.lib()
    dev = torch.device("cuda:0")
    if args.probe:
        probe(nne, torch, dev)
        return

    b, hq, hkv, t, d = 4, 32, 8, 2048, 128
    q, k, v = config2_inputs(torch, dev)
    out = torch.empty_like(q)
    print("bench: config2 prefill steps=%d warmup=%d" % (args.steps, args.warmup),
          file=sys.stderr, flush=True)
    # Untimed, before the warm-up steps: bring the GPU to its working clocks.
    settle_ms = settle_clocks(torch, lambda: nne.attention_forward(q, k, v, True, out=out))
    ms, kms = time_prefill(nne, torch, q, k, v, True, args.steps, args.warmup, out)
    flops = causal_flops(b, hq, t, d)
    value = flops / (ms / 1e3) / 1e12
    achieved = flops / (kms / 1e3) / 1e12
    line = {
        "metric": "prefill attn TFLOP/s + decode KV-read GB/s on 1 MI355X, vs host-CPU Rayon",
        "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "clock_settle_ms": round(settle_ms, 1),
        "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config2: GQA causal prefill B=4 Hq=32 Hkv=8 T=2048 d=128 f32, "
                               "Q/K/V~N(0,1), per-position scale U[0.5,1.5] on Q,K",
                   "global_batch": b, "seq_len": t, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_MATRIX_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MATRIX_TFLOPS, 4),
                     "traffic": TRAFFIC_PREFILL_CONFIG2,
                     "kernel": "prefill_mfma_kernel<128, true, true, false>",
                     "kernel_ms": round(kms, 4)},
    }
    del q, k, v, out
    # CPU legs run after every GPU measurement: an idle GPU drops its clocks,
    # and a launch timed right after seconds of host work would pay the ramp.
    cpu_jobs = []
    if not args.no_decode:
        print("bench: config3 decode", file=sys.stderr, flush=True)
        line["decode"] = bench_decode(nne, torch, dev, traffic=TRAFFIC_DECODE_CONFIG3_STEP)
        if not args.no_cpu:
            cpu_jobs.append((line["decode"], decode_cpu_baseline))
    if not args.headline:
        extra = []
        g = torch.Generator(device=dev).manual_seed(0x5EED0001)
        for name, (bb, h, tt, dd, causal, std) in {
            "config1": (1, 4, 256, 64, True, 1.0),
            "config4": (1, 16, 16384, 64, True, 0.5),
            "config5a": (8, 20, 1500, 64, False, 1.0),
            "d256": (1, 16, 4096, 256, True, 1.0),
            "d512": (1, 16, 4096, 512, True, 1.0),
        }.items():
            q = torch.randn(bb, h, tt, dd, generator=g, device=dev) * std
            k = torch.randn(bb, h, tt, dd, generator=g, device=dev) * std
            v = torch.randn(bb, h, tt, dd, generator=g, device=dev) * std
            o = torch.empty_like(q)
            ms_c, kms_c = time_prefill(nne, torch, q, k, v, causal, max(3, args.steps // 2), 2, o)
            fl = causal_flops(bb, h, tt, dd) if causal else full_flops(bb, h, tt, tt, dd)
            rec = {"workload": {
                "d256": "d256: causal prefill, head dim 256 (wave-pair kernel), B=1 H=16 T=4096 f32",
                "d512": "d512: causal prefill, head dim 512 (deep kernel), B=1 H=16 T=4096 f32",
            }.get(name, name)}
            if name == "config1":
                # A ~15 us call: host-paced events measure Python's issue
                # rate, so the device rate is taken with the calls queued.
                paced = kms_c
                kms_c = gpu_ms_per_call(
                    torch, lambda i: nne.attention_forward(q, k, v, causal, out=o), 50, True)
                rec["host_paced_kernel_ms"] = round(paced, 4)
                # The floor any launch pays: an (almost) empty kernel, queued the same way.
                rec["empty_kernel_ms"] = round(gpu_ms_per_call(
                    torch, lambda i: torch.cuda._sleep(1), 50, True), 4)
            ach = fl / (kms_c / 1e3) / 1e12
            rec.update({"TFLOP/s": round(ach, 3), "kernel_ms": round(kms_c, 4),
                        "frac": round(ach / PEAK_FP32_MATRIX_TFLOPS, 4),
                        "roofline": {"bound": "mfma", "achieved": round(ach, 3),
                                     "peak": PEAK_FP32_MATRIX_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(ach / PEAK_FP32_MATRIX_TFLOPS, 4),
                                     "flops": fl,
                                     "traffic": {"config1": TRAFFIC_PREFILL_CONFIG1,
                                                 "config4": TRAFFIC_PREFILL_CONFIG4,
                                                 "config5a": TRAFFIC_PREFILL_CONFIG5A,
                                                 "d256": TRAFFIC_PREFILL_D256,
                                                 "d512": TRAFFIC_PREFILL_D512}[name]}})
            if not args.no_cpu:
                # Bounded samples of the same workload (a few seconds each).
                cpu_jobs.append((rec, {
                    "config1": lambda: flash_cpu_baseline(1, 4, 256, 64, True, 1.0,
                                                          "config 1 in full (B=1, H=4, T=256, d=64)",
                                                          reps=5),
                    "config4": lambda: flash_cpu_baseline(1, 16, 4096, 64, True, 0.5,
                                                          "config 4 at a quarter of its length "
                                                          "(B=1, H=16, T=4096, d=64)"),
                    "config5a": lambda: flash_cpu_baseline(1, 20, 1500, 64, False, 1.0,
                                                           "one of the 8 batch elements of "
                                                           "config 5a (H=20, T=1500, d=64)"),
                    "d256": lambda: flash_cpu_baseline(1, 16, 2048, 256, True, 1.0,
                                                       "the d = 256 line at half its length "
                                                       "(B=1, H=16, T=2048, d=256)"),
                    "d512": lambda: flash_cpu_baseline(1, 16, 1024, 512, True, 1.0,
                                                       "the d = 512 line at a quarter of its "
                                                       "length (B=1, H=16, T=1024, d=512)"),
                }[name]))
            extra.append(rec)
            if name == "config5a":
                # Three K/V sets (369 MB) rotated so no call finds its K/V in
                # the 256 MB MALL.
                qx = torch.randn(8, 20, 8, 64, generator=g, device=dev)
                ox = torch.empty_like(qx)
                kvs = [(k, v)] + [(torch.randn_like(k), torch.randn_like(v)) for _ in range(2)]
                for i in range(3):
                    nne.attention_forward(qx, kvs[i][0], kvs[i][1], False, out=ox)
                reps = 30
                call = lambda i: nne.attention_forward(qx, kvs[i % 3][0], kvs[i % 3][1], False,
                                                       out=ox)
                kms_x = gpu_ms_per_call(torch, call, reps, queued=True)
                hms_x = gpu_ms_per_call(torch, call, reps, queued=False)
                by = (2 * 8 * 20 * 1500 * 64 + 2 * 8 * 20 * 8 * 64) * 4
                gbs_x = by / (kms_x / 1e3) / 1e9
                extra.append({"workload": "config5b cross 8q->1500", "GB/s":
                              round(gbs_x, 1), "kernel_ms": round(kms_x, 4),
                              "frac": round(gbs_x / PEAK_HBM_GBS, 4),
                              "roofline": {"bound": "hbm", "achieved": round(gbs_x, 1),
                                           "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                           "frac": round(gbs_x / PEAK_HBM_GBS, 4), "bytes": by,
                                           "traffic": TRAFFIC_CROSS_CONFIG5B},
                              "host_paced_GB/s": round(by / (hms_x / 1e3) / 1e9, 1),
                              "note": "3 K/V sets rotated (369 MB > 256 MB MALL); calls queued "
                                      "behind a spin kernel so the GPU runs them back to back; "
                                      "host_paced = issued from Python one by one"})
                if not args.no_cpu:
                    cpu_jobs.append((extra[-1], cross_cpu_baseline))
                del kvs
            del q, k, v, o
        print("bench: G=8 decode", file=sys.stderr, flush=True)
        rec = bench_decode(nne, torch, dev, hq=64, seed=0x5EED0016,
                           workload="G=8 decode (LLaMA-2-70B grouping): B=32 Hq=64 Hkv=8 d=128 "
                                    "L0~U[512,4096] ragged, 64 steps append+attend, f32",
                           traffic=TRAFFIC_DECODE_G8_STEP)
        rec["workload"] = rec["config"]["workload"]
        extra.append(rec)
        if not args.no_cpu:
            cpu_jobs.append((rec, lambda: decode_cpu_baseline(
                seed=0x5EED0016, shape=(32, 64, 8, 128), label="G=8 decode step")))
        print("bench: config3 decode layer step", file=sys.stderr, flush=True)
        extra.append(bench_decode_layer(nne, torch, dev))
        if not args.no_cpu:
            cpu_jobs.append((extra[-1], prologue_cpu_baseline))
        print("bench: MHA decode layer step", file=sys.stderr, flush=True)
        extra.append(bench_mha_decode_layer(nne, torch, dev))
        if not args.no_cpu:
            cpu_jobs.append((extra[-1], lambda: decode_cpu_baseline(
                seed=0x5EED0015, n_seq=32, steps=4, shape=(32, 12, 12, 64), len_range=(128, 1024),
                label="GPT-2-small MHA decode attend", mode="mha")))
        line["other_configs"] = extra
    if not args.no_cpu:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        for rec, job in cpu_jobs:
            rec["cpu_baseline"] = job()
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
