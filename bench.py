"""Benchmark of the cache-aware streaming FastConformer encoder step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload chunk2|chunk14|chunk2x1024|decode|decode_mq|offline|rnnt|stream|stream14]
                    [--no-cpu-baseline]

A step is one cache-aware encoder chunk step for every stream of the batch: the mel chunk (new rows
plus the 9-row pre-encode cache) through the causal dw_striding 8x subsampling with 2 frames dropped,
then 24 conformer layers (bf16-valued weights held as IEEE half; half activations, K/V caches and
MFMA operands; fp32 accumulation), with inputs already in HBM and full 70-frame caches seeded from
N(0,1).  Default workload: 64 streams x 2 frames (25 mel rows in, 160 ms of audio per stream per
step).  Prints one JSON line: aggregate streamed audio-seconds per second, per-step latency
percentiles, the fused attention kernel's achieved HBM bandwidth against 8 TB/s and against the HBM
read peak measured in the same run (HIP events on the kernel's own stream), each projection GEMM's
MFMA throughput against the nominal and the measured peak, and the CPU oracle's throughput on a
bounded sample timed on this host's cores; then the other configurations' figures: the long-chunk
workload (256 streams x 14 frames) -- its attention kernel (roofline_long_chunk), its whole step
and its projections' MFMA use (chunk14_step) -- the offline attention kernel's MFMA fraction
(offline_attention) and the paged decode attention's HBM fraction (decode_attention).
--library-gemm adds the vendor GEMM (torch.matmul, hipBLASLt) timed on each projection's shape.

--workload chunk14 runs the same step at 256 streams x 14 frames.  --workload decode measures the
decoder's paged grouped-query attention instead: 64 sequences x 1 new token, 32 query / 8 kv heads
x 128, contexts uniform in 512..4096 keys in bf16 pages of 16 (one line in the same format, value in
tokens/s); --workload decode_mq the same with 4 new positions per sequence in one multi-query call.  --workload offline measures the whole-utterance rel-pos attention: 8 utterances x 1500
frames, 8 heads x 128, valid lengths uniform in 900..1500 as key padding (value in frames/s, roofline
against the bf16 MFMA peak).  --workload rnnt measures the joint.enc projection and greedy RNN-T
decoding of 64 streams x 2 frames per chunk.  --workload stream measures live transcription end to
end through the batched streamer: 64 streams x 160 ms of audio pushed per step, mel frontend,
subsampling, 24 layers, joint.enc and greedy RNN-T (value in audio-sec/sec, audio in to tokens out).
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
FRAME_SEC = 0.08          # one encoder frame after 8x subsampling of 10 ms mel hops
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, vendor nominal

WORKLOADS = {
    "chunk2": dict(streams=64, T=2),     # 64 concurrent streams, 160 ms chunks
    "chunk14": dict(streams=256, T=14),  # 256 concurrent streams, 1120 ms chunks
    "chunk2x1024": dict(streams=1024, T=2),  # the 160 ms chunk at 1024 concurrent streams
    "decode": dict(seqs=64, q_heads=32, kv_heads=8, head_dim=128, page=16, ctx=(512, 4096)),
    # the same cache with 4 new positions per sequence (one multi-query call)
    "decode_mq": dict(seqs=64, q_heads=32, kv_heads=8, head_dim=128, page=16, ctx=(512, 4096), queries=4),
    "offline": dict(batch=8, frames=1500, heads=8, head_dim=128, valid=(900, 1500)),
    "rnnt": dict(streams=64, T=2, hidden=640, vocab=1025, layers=2),
    "stream": dict(streams=64, lookahead=1),     # live audio -> tokens, 160 ms chunks
    "stream14": dict(streams=256, lookahead=13), # live audio -> tokens, 1120 ms chunks
}
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def load_pkg():
    name = "universal_dictator_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "universal-dictator_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def read_traffic(kernel_tag):
    """HBM bytes per launch of a kernel from a committed rocprofv3 --pmc summary
    (profiles/<tag>_traffic.md, line 'traffic_bytes_per_launch: N'), or None."""
    path = os.path.join(ROOT, "profiles", kernel_tag + "_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def host_cpu():
    """The host's CPUs as this job sees them: model, nproc, the CPUs in this process's affinity
    mask, the physical cores among them, the cgroup CPU quota, and the OpenMP thread count the
    environment grants (OMP_NUM_THREADS).  The baseline uses every physical core the job may run
    on: the smallest of the affine physical cores, the quota and the granted thread count."""
    info = {"model": None, "nproc": os.cpu_count()}
    cores = {}
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = [x.strip() for x in line.split(":", 1)]
                cur[k] = v
                if k == "model name" and info["model"] is None:
                    info["model"] = v
            elif cur:
                if "processor" in cur:
                    cores[int(cur["processor"])] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
                cur = {}
        if cur and "processor" in cur:
            cores[int(cur["processor"])] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
    except OSError:
        pass
    aff = sorted(os.sched_getaffinity(0))
    info["affinity_cpus"] = len(aff)
    info["affinity_physical_cores"] = len({cores[c] for c in aff if c in cores}) or len(aff)
    quota = None
    try:
        q, per = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) / int(per)))
    except (OSError, ValueError):
        pass
    info["cgroup_cpu_quota"] = quota
    granted = os.environ.get("OMP_NUM_THREADS")
    info["omp_num_threads_env"] = int(granted) if granted and granted.isdigit() else None
    threads = info["affinity_physical_cores"]
    for lim in (quota, info["omp_num_threads_env"]):
        if lim:
            threads = min(threads, lim)
    info["threads"] = max(1, threads)
    return info


def load_oracle(threads):
    """The oracle (test infrastructure, the CPU baseline here), with OpenMP threads bound close to
    one physical core each; the binding is read when the OpenMP runtime loads with the oracle."""
    os.environ["OMP_PROC_BIND"] = "close"
    os.environ["OMP_PLACES"] = "cores"
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    orc.set_threads(threads)
    return orc


def timed_median(fn, budget_s, min_steps=5, max_steps=60, warm=1):
    """Median seconds of fn over >= min_steps timed calls after `warm` untimed ones, until about
    budget_s has passed; returns (median, n, total seconds)."""
    for _ in range(warm):
        fn()
    ts = []
    t_all = time.perf_counter()
    while len(ts) < min_steps or (time.perf_counter() - t_all < budget_s and len(ts) < max_steps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts), time.perf_counter() - t_all


def cpu_baseline(lw, sw, cfg, S, T, budget_s, cpu, S_sample=None):
    """The oracle's encodeStreamStep (fp32, OpenMP) on this host: whole steps of the same workload
    (subsampling of every stream's mel chunk, then all layers) over S_sample of the S streams (all
    when None), the median of >= 5 timed steps after one warm-up step."""
    threads = cpu["threads"]
    orc = load_oracle(threads)
    Sn = S_sample or S
    model = orc.Model(lw, cfg.d_model, cfg.heads, cfg.ff_dim, cfg.conv_kernel)
    model.prepare(-(T - 1), cfg.left_context + T - 1)
    rng = np.random.default_rng(5)
    L, D = cfg.left_context, cfg.d_model
    kc = rng.standard_normal((Sn, cfg.layers, L, D), dtype=np.float32)
    vc = rng.standard_normal((Sn, cfg.layers, L, D), dtype=np.float32)
    cc = rng.standard_normal((Sn, cfg.layers, cfg.conv_kernel - 1, D), dtype=np.float32)
    cl = np.full(Sn, L, np.int32)
    rows = mel_rows(T)
    mel = rng.standard_normal((Sn, rows, 128), dtype=np.float32)
    valid = np.full(Sn, T, np.int32)

    def step():
        x = np.stack([orc.subsample(mel[s], rows, sw)[2:] for s in range(Sn)])
        orc.stream_step(model, x, valid, kc, vc, cc, cl)

    med, n, el = timed_median(step, budget_s)
    return dict(value=round(Sn * T * FRAME_SEC / med, 3), unit="audio-sec/sec", cores=threads, kind="port",
                threads=threads, cpu_model=cpu["model"], nproc=cpu["nproc"], affinity_cpus=cpu["affinity_cpus"],
                affinity_physical_cores=cpu["affinity_physical_cores"], cgroup_cpu_quota=cpu["cgroup_cpu_quota"],
                omp_num_threads_env=cpu["omp_num_threads_env"], omp_proc_bind="close", statistic="median",
                sample="%s%d streams x %d mel rows -> %d frames, %d layers, fp32: median of %d whole steps "
                       "(after 1 warm-up), %.3f s/step, %.1f s in all"
                       % ("%d of the " % Sn if Sn != S else "", S, rows, T, cfg.layers, n, med, el))


def warm_up(fn, hs, min_calls, min_ms=150.0):
    """Untimed calls until at least min_calls have run and min_ms of wall time has passed, waiting
    for the stream every 10 calls.  Under sustained load the GPU's clock rises over the first
    ~30-40 ms (the offline attention launch takes 214 us at first and 157 us from ~35 ms on; a
    256-stream x 14-frame step 8.4 ms at first and 7.9 ms after 60 ms), so the figures that follow
    are of the steady state.  Returns the number of calls run."""
    n, t0 = 0, time.perf_counter()
    while n < min_calls or (time.perf_counter() - t0) * 1000.0 < min_ms:
        for _ in range(10):
            fn()
        n += 10
        hs.synchronize()
    return n


def mel_rows(T):
    """Mel rows of a chunk that yields T encoder frames after the 2 dropped ones: 8 (T + 2) - 7
    (16 new rows + 9 pre-encode cache rows for T = 2, NemotronSchedule.swift)."""
    return 8 * (T + 2) - 7


def decode_bench(ud, args, summary=False, steps=None, warmup=None, workload="decode"):
    """Paged GQA decode attention: one new token for each of 64 sequences (workload decode), or 4
    new positions per sequence in one multi-query call (decode_mq).  summary: return the kernel's
    figures as a dict (no CPU baseline, nothing printed) for the default line."""
    steps = steps or args.steps
    warmup = args.warmup if warmup is None else warmup
    wl = WORKLOADS[workload]
    n, Hq, Hkv, d, page = wl["seqs"], wl["q_heads"], wl["kv_heads"], wl["head_dim"], wl["page"]
    M = wl.get("queries", 1)
    rng = np.random.default_rng(17)
    lens = rng.integers(wl["ctx"][0], wl["ctx"][1] + 1, n)
    nb = (lens + page - 1) // page
    max_blocks = (wl["ctx"][1] + page - 1) // page
    nblk = int(nb.sum())
    perm = rng.permutation(nblk).astype(np.int32)
    table = np.zeros((n, max_blocks), np.int32)
    o = 0
    for i in range(n):
        table[i, :nb[i]] = perm[o:o + nb[i]]
        o += nb[i]
    log("device %s; workload %s: %d sequences x %d queries, %d/%d heads x %d, context %d..%d (total %d keys), "
        "bf16 pages of %d" % (ud.device_arch(), workload, n, M, Hq, Hkv, d, lens.min(), lens.max(), lens.sum(), page))

    def pages():
        x = rng.standard_normal((nblk, Hkv, page, d), dtype=np.float32)
        return (ud.round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)
    kp_h, vp_h = pages(), pages()
    kp, vp = ud.DeviceBuffer.from_numpy(kp_h), ud.DeviceBuffer.from_numpy(vp_h)
    q_h = rng.standard_normal((n, M, Hq * d), dtype=np.float32)
    q = ud.DeviceBuffer.from_numpy(q_h)
    # query m of a sequence of L keys: keys [0, L - (M - 1) + m) (causal over the M new positions)
    ranges_h = np.zeros((n, M, 2), np.int32)
    for m in range(M):
        ranges_h[:, m, 1] = lens - (M - 1) + m
    ranges = ud.DeviceBuffer.from_numpy(ranges_h)
    tbl = ud.DeviceBuffer.from_numpy(table)
    max_keys = int(lens.max())
    ws = ud.DeviceBuffer.zeros(ud.gqa_workspace_bytes(n * M, Hq, d, max_keys))
    out = ud.DeviceBuffer(n * M * Hq * d * 4)
    hs = ud.HipStream()
    if M == 1:
        call = lambda: ud.gqa_attention_paged(q, kp, vp, tbl, max_blocks, ranges, out, n, Hq, Hkv, d, max_keys, ws,
                                              hip_stream=hs)
    else:
        call = lambda: ud.gqa_attention_paged_mq(q, kp, vp, tbl, max_blocks, ranges, out, n, M, Hq, Hkv, d, max_keys,
                                                 ws, hip_stream=hs)
    warmed = warm_up(call, hs, warmup)
    e0, e1 = ud.Event(), ud.Event()
    e0.record(hs)
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    e1.record(hs)
    e1.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0
    ms = max(wall_ms, e0.elapsed_ms(e1)) / steps
    kv_bytes = int(lens.sum()) * Hkv * d * 2 * 2
    algo = kv_bytes + n * M * Hq * d * 4 * 2 + int(nb.sum()) * 4 + n * M * 8
    achieved = algo / (ms / 1000.0) / 1e9
    log("timed %d calls: %.2f us per decode attention step (split + combine), %.0f GB/s" % (steps, ms * 1000, achieved))
    if summary:
        return {"kernel": "gqa_split_mfma_kernel + gqa_combine_kernel (timed together)",
                "workload": "%d sequences x %d token%s, %d query / %d kv heads x %d, context %d..%d, bf16 pages of %d"
                            % (n, M, "s" if M > 1 else "", Hq, Hkv, d, wl["ctx"][0], wl["ctx"][1], page),
                "us_per_call": round(ms * 1000.0, 3), "tokens_per_sec": round(n * M / (ms / 1000.0), 1),
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_call": algo,
                "calls_timed": steps, "warmup_calls": warmed}
    result = {
        "metric": "paged GQA decode attention: tokens/s and HBM roofline fraction",
        "value": round(n * M / (ms / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warmed, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 K/V pages, fp32 queries, softmax and accumulation (bf16 MFMA operands)",
        "data": "synthetic (seeded N(0,1) queries and bf16 K/V pages, random page table)",
        "config": {"workload": "decode-step grouped-query attention over a paged K/V cache, %d sequences x %d "
                               "token%s, %d query / %d kv heads x %d, context %d..%d, pages of %d"
                               % (n, M, "s" if M > 1 else "", Hq, Hkv, d, wl["ctx"][0], wl["ctx"][1], page),
                   "sequences": n, "queries_per_sequence": M, "q_heads": Hq, "kv_heads": Hkv, "head_dim": d,
                   "total_keys": int(lens.sum())},
        "roofline": {"kernel": "gqa_split_mfma_kernel + gqa_combine_kernel (timed together)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic("gqa_decode" if M == 1 else "gqa_decode_mq"),
                     "algorithmic_bytes_per_launch": algo},
    }
    if not args.no_cpu_baseline:
        cpu = host_cpu()
        threads = cpu["threads"]
        orc = load_oracle(threads)
        log("cpu baseline: oracle attention on %d threads, ~%.0f s" % (threads, args.cpu_seconds))
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds and done < n:
            i = done
            rows = lambda pg: pg[table[i, :nb[i]]].transpose(0, 2, 1, 3).reshape(-1, Hkv * d)[:lens[i]]
            k = (rows(kp_h).astype(np.uint32) << 16).view(np.float32)
            v = (rows(vp_h).astype(np.uint32) << 16).view(np.float32)
            orc.gqa_attention(q_h[i], k, v, ranges_h[i], Hq, Hkv)
            done += 1
        el = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(done * M / el, 3), "unit": "tokens/s", "cores": threads,
                                  "kind": "port", "cpu_model": cpu["model"], "nproc": cpu["nproc"],
                                  "omp_proc_bind": "close",
                                  "sample": "%d of the %d sequences (%d token%s each, all heads) in %.1f s, "
                                            "including the page gather" % (done, n, M, "s" if M > 1 else "", el)}
    print(json.dumps(result), flush=True)


def offline_bench(ud, args, summary=False, steps=None, warmup=None):
    """Offline rel-pos attention over a padded batch of whole utterances (one launch = one layer).
    summary: return the kernel's figures as a dict (no CPU baseline, nothing printed)."""
    steps = steps or args.steps
    warmup = args.warmup if warmup is None else warmup
    wl = WORKLOADS["offline"]
    B, T, H, dk = wl["batch"], wl["frames"], wl["heads"], wl["head_dim"]
    D = H * dk
    rng = np.random.default_rng(23)
    lens = rng.integers(wl["valid"][0], wl["valid"][1] + 1, B)
    log("device %s; workload offline: %d utterances x %d frames, valid %s, %d heads x %d, bf16"
        % (ud.device_arch(), B, T, [int(x) for x in lens], H, dk))
    bits = lambda a: (ud.round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)
    q, k, v = (ud.DeviceBuffer.from_numpy(bits(rng.standard_normal((B, T, D), dtype=np.float32))) for _ in range(3))
    n_rel = 2 * T - 1
    P = ud.DeviceBuffer.from_numpy(bits((rng.standard_normal((n_rel, D)) * 0.5).astype(np.float32)))
    u = ud.DeviceBuffer.from_numpy((rng.standard_normal((H, dk)) * 0.02).astype(np.float32))
    vb = ud.DeviceBuffer.from_numpy((rng.standard_normal((H, dk)) * 0.02).astype(np.float32))
    # key padding: full context is one chunk of T frames, clipped to each utterance's valid length
    ranges_h = ud.chunked_limited_ranges(T, T, T - 1, valid=lens)
    ranges = ud.DeviceBuffer.from_numpy(ranges_h)
    out = ud.DeviceBuffer(B * T * D * 2)
    hs = ud.HipStream()
    call = lambda: ud.rel_pos_attention_batched(q, k, v, P, T - 1, u, vb, ranges, out, B, T, H, n_rel, hip_stream=hs)
    warmed = warm_up(call, hs, warmup)
    e0, e1 = ud.Event(), ud.Event()
    e0.record(hs)
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    e1.record(hs)
    e1.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0
    ms = max(wall_ms, e0.elapsed_ms(e1)) / steps
    flops_dense = 6.0 * B * H * T * T * dk               # ac + bd + P.V over the padded T x T
    flops_valid = 6.0 * H * T * float(lens.sum()) * dk   # keys limited to each utterance's valid frames
    tflops = flops_dense / (ms / 1000.0) / 1e12
    log("timed %d launches: %.2f us each, %.1f TFLOP/s dense-equivalent (%.1f on valid keys)"
        % (steps, ms * 1000, tflops, flops_valid / (ms / 1000.0) / 1e12))
    if summary:
        return {"kernel": "relpos_dense_kernel",
                "workload": "%d utterances x %d frames, %d heads x %d, key padding %d..%d, bf16"
                            % (B, T, H, dk, wl["valid"][0], wl["valid"][1]),
                "us_per_launch": round(ms * 1000.0, 3), "frames_per_sec": round(B * T / (ms / 1000.0), 1),
                "bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_launch": flops_dense,
                "valid_key_tflops": round(flops_valid / (ms / 1000.0) / 1e12, 2), "launches_timed": steps,
                "warmup_launches": warmed}
    result = {
        "metric": "offline rel-pos attention: frames/s and bf16 MFMA roofline fraction",
        "value": round(B * T / (ms / 1000.0), 1),
        "unit": "frames/s (one layer, all heads)",
        "n_gpus": 1, "steps": steps, "warmup": warmed, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 q/k/v/P operands, fp32 softmax and accumulation",
        "data": "synthetic (seeded N(0,1) q/k/v, random position table, random valid lengths)",
        "config": {"workload": "offline full-context rel-pos MHSA, %d utterances x %d frames (%d s), %d heads x %d, "
                               "key padding %d..%d" % (B, T, int(T * FRAME_SEC), H, dk, wl["valid"][0], wl["valid"][1]),
                   "batch": B, "frames": T, "heads": H, "head_dim": dk, "valid_lengths": [int(x) for x in lens]},
        "roofline": {"kernel": "relpos_dense_kernel", "bound": "mfma", "achieved": round(tflops, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": read_traffic("relpos_dense_offline"),
                     "algorithmic_flops_per_launch": flops_dense, "valid_key_flops_per_launch": flops_valid},
    }
    if not args.no_cpu_baseline:
        cpu = host_cpu()
        threads = cpu["threads"]
        orc = load_oracle(threads)
        log("cpu baseline: oracle attention on %d threads, ~%.0f s" % (threads, args.cpu_seconds))
        qh = ud.round_bf16(rng.standard_normal((T, D)).astype(np.float32))
        kh = ud.round_bf16(rng.standard_normal((T, D)).astype(np.float32))
        Ph = ud.round_bf16(rng.standard_normal((n_rel, D)).astype(np.float32))
        uh = np.zeros((H, dk), np.float32)
        rows, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds and rows < T:
            sel = np.zeros((T, 2), np.int32)
            sel[rows:rows + 64] = [0, int(lens[0])]
            orc.relpos_attention(qh, kh, kh, Ph, uh, uh, sel, T - 1, H)
            rows += 64
        el = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(rows / el, 2), "unit": "frames/s (one layer, all heads)",
                                  "cores": threads, "kind": "port", "cpu_model": cpu["model"], "nproc": cpu["nproc"],
                                  "omp_proc_bind": "close",
                                  "sample": "%d query frames of one %d-frame utterance (%d valid keys) in %.1f s"
                                            % (rows, T, lens[0], el)}
    print(json.dumps(result), flush=True)


def rnnt_bench(ud, args):
    """joint.enc projection + greedy RNN-T decode of 64 streams x 2 encoder frames per chunk (the
    step after the encoder, Nemotron.swift:82-90 + RNNT.swift:125-151), timed at the two emission
    extremes: every frame blank (one joint per frame, the cached prediction reused) and every frame
    at the 10-symbol cap (a prediction and a joint per symbol); and in between, a joint whose blank
    bias lets some frames emit a few symbols (later greedy iterations then have a few active
    streams).  value: audio-sec/sec of the all-blank regime."""
    wl = WORKLOADS["rnnt"]
    S, T = wl["streams"], wl["T"]
    log("device %s; workload rnnt: %d streams x %d frames, hidden %d, vocab %d, %d LSTM layers, fp32"
        % (ud.device_arch(), S, T, wl["hidden"], wl["vocab"], wl["layers"]))
    rng = np.random.default_rng(3)
    enc = ud.DeviceBuffer.from_numpy(rng.standard_normal((S * T, 1024), dtype=np.float32))
    proj = ud.DeviceBuffer(S * T * wl["hidden"] * 4)
    hs = ud.HipStream()
    res = {}
    for regime, bias in (("blank", 50.0), ("cap", -50.0), ("mixed", 1.0)):
        r = ud.Rnnt(max_streams=S)
        r.set_weights(ud.synthetic_rnnt_weights(7, blank_bias=bias))
        slots = list(range(S))

        def chunk():
            r.project(S * T, enc, proj, hip_stream=hs)
            return r.greedy(slots, proj, T, [T] * S, cap=32, hip_stream=hs)[1]

        for _ in range(max(2, args.warmup // 4)):
            chunk()
        steps = max(5, args.steps // 10)
        t0 = time.perf_counter()
        toks = 0
        for _ in range(steps):
            toks += int(chunk().sum())
        ms = (time.perf_counter() - t0) * 1000.0 / steps
        res[regime] = (ms, toks / steps)
        log("%s regime: %.3f ms per chunk, %.1f tokens per chunk" % (regime, ms, toks / steps))
        r.close()
    ms = res["blank"][0]
    result = {
        "metric": "aggregate audio-sec/sec of joint + greedy RNN-T decoding at 64 streams",
        "value": round(S * T * FRAME_SEC / (ms / 1000.0), 2),
        "unit": "audio-sec/sec",
        "n_gpus": 1, "steps": max(5, args.steps // 10), "warmup": max(2, args.warmup // 4),
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded random-init prediction/joint weights, N(0,1) encoder rows)",
        "config": {"workload": "joint.enc + greedy RNN-T, %d streams x %d frames per chunk, all frames blank" % (S, T),
                   "streams": S, "frames": T, "hidden": wl["hidden"], "vocab": wl["vocab"], "layers": wl["layers"]},
        "cap_regime_ms_per_chunk": round(res["cap"][0], 4),
        "cap_regime_tokens_per_chunk": res["cap"][1],
        "mixed_regime_ms_per_chunk": round(res["mixed"][0], 4),
        "mixed_regime_tokens_per_chunk": res["mixed"][1],
    }
    print(json.dumps(result), flush=True)


# (regime, blank logit bias of the synthetic joint) per workload: every frame blank, every frame
# at the 10-symbol cap, and a mixed rate near speech (stream: 0.2-0.7 tokens per 160 ms
# stream-chunk, stream14: about 6.6 per 1120 ms chunk, i.e. 1.4-6 tokens/s, depending on the audio
# the timed steps push).  The synthetic joint's blank margin is nearly the same on every frame, so
# the rate falls from the cap to none within a few hundredths of bias, and the tokens gather on
# few streams: the greedy loop, which runs as many iterations as the busiest stream needs, costs
# more at a given mean rate than a trained joint's spread emissions would.
STREAM_REGIMES = {
    "stream": (("blank", 50.0), ("cap", -50.0), ("mixed", 1.24)),
    "stream14": (("blank", 50.0), ("cap", -50.0), ("mixed", 1.16)),
}


def stream_bench(ud, args):
    """Live transcription end to end through the batched streamer (include/ud_streamer.h): every
    timed step pushes one chunk of new samples to each stream (stream: 64 streams x 2560 samples =
    160 ms; stream14: 256 streams x 17920 samples = 1120 ms), which completes one chunk per stream
    and runs one batched step: sample staging + H2D, the mel kernel (the chunk's frames plus the 9
    pre-encode frames, recomputed), subsampling, 24 bf16 layers, joint.enc and greedy RNN-T with
    its host readbacks.  Caches are full before timing.  A random-init joint emits on every frame
    or on none, so the decoder is timed at both ends, as in the rnnt workload: every frame blank
    (value) and every frame at the 10-symbol cap, and in between at a speech-like mean rate.
    value: audio-sec/sec end to end."""
    wl = WORKLOADS[args.workload]
    S, la = wl["streams"], wl["lookahead"]
    T = la + 1
    hop = 160 * 8 * T
    cfg = ud.EncoderConfig(layers=24, max_chunk=T, max_streams=S, dtype="bf16")
    log("device %s; workload %s: %d live streams, lookahead %d (%d ms chunks), 24 layers bf16"
        % (ud.device_arch(), args.workload, S, la, int(T * FRAME_SEC * 1000)))
    enc = ud.Encoder(cfg)
    for l in range(cfg.layers):
        enc.set_layer_weights(l, ud.synthetic_layer_weights(cfg, 2024, l, ln_jitter=0.0))
    enc.set_subsampling_weights(ud.synthetic_subsampling_weights(2025))
    enc.finalize()
    # a Slaney-like triangular filterbank and a symmetric Hann window (the checkpoint's buffers
    # are of this form)
    fb = np.zeros((128, 257), np.float32)
    edges = np.linspace(1, 256, 130)
    k = np.arange(257)
    for m in range(128):
        lo, mid, hi = edges[m], edges[m + 1], edges[m + 2]
        fb[m] = np.clip(np.minimum((k - lo) / (mid - lo), (hi - k) / (hi - mid)), 0, None) * (2.0 / (hi - lo))
    win = (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(400) / 399)).astype(np.float32)
    fe = ud.MelFrontend(fb, win)
    rng = np.random.default_rng(5)
    n_src = 16000 * 12
    t = np.arange(n_src) / 16000.0
    srcs = []
    for b in range(S):
        f0 = 100 + 60 * rng.random() + 30 * np.sin(2 * np.pi * 0.5 * t + b)
        ph = 2 * np.pi * np.cumsum(f0) / 16000.0
        x = sum(np.sin(h * ph) / h for h in range(1, 9)) * (0.2 + 0.15 * np.sin(2 * np.pi * 1.1 * t + b))
        srcs.append((0.3 * x + 0.003 * rng.standard_normal(n_src)).astype(np.float32))
    # ud_mel_features alone at the streamer's launch shape (S jobs x (9 + 8T) frames), HIP events on
    # its stream: the job-list copy and the kernel
    hs = ud.HipStream()
    rows = 9 + 8 * T
    clip = (rows - 1) * 160
    ab = ud.DeviceBuffer.from_numpy(np.stack([s[:clip] for s in srcs]))
    mb = ud.DeviceBuffer(S * rows * 128 * 4)
    for _ in range(5):
        fe.features_device(S, ab, clip, [clip] * S, mb, rows, hip_stream=hs)
    e0, e1 = ud.Event(), ud.Event()
    e0.record(hs)
    for _ in range(50):
        fe.features_device(S, ab, clip, [clip] * S, mb, rows, hip_stream=hs)
    e1.record(hs)
    e1.synchronize()
    mel_us = e0.elapsed_ms(e1) * 1000.0 / 50
    log("mel call (job-list copy + kernel): %.1f us per step (%d streams x %d frames)" % (mel_us, S, rows))
    warm = max(args.warmup, 40) if T <= 2 else max(args.warmup // 4, 8)
    res = {}
    for regime, bias in STREAM_REGIMES[args.workload]:
        dec = ud.Rnnt(max_streams=S)
        dec.set_weights(ud.synthetic_rnnt_weights(2026, blank_bias=bias))
        st = ud.Streamer(enc, dec, fe, lookahead=la, max_streams=S)
        ids = [st.open() for _ in range(S)]
        pos = [0]

        def piece(first):
            n = (8 * la + 1) * 160 + 40 if first else hop    # exactly completes the next chunk
            out = {}
            for b in range(S):
                a = pos[0] % (n_src - n)
                out[ids[b]] = srcs[b][a:a + n]
            pos[0] += n
            return out

        st.push(piece(True))
        for _ in range(warm):
            st.push(piece(False))
        steps = (args.steps if regime != "cap" else max(5, args.steps // 5)) if T <= 2 else \
            (max(10, args.steps // 5) if regime != "cap" else 5)
        b0, c0 = st.stats()
        tok0 = sum(len(st.tokens(i)) for i in ids)
        # each step's push arguments packed ahead (a C or Swift caller passes its pointers as they are)
        pieces = [ud.Streamer.Pushed(piece(False)) for _ in range(steps)]
        ud.synchronize()
        t0 = time.perf_counter()
        for p in pieces:
            st.push(p)
        wall = time.perf_counter() - t0
        b1, c1 = st.stats()
        toks = sum(len(st.tokens(i)) for i in ids) - tok0
        if b1 - b0 != steps or c1 - c0 != steps * S:
            raise RuntimeError("expected one batched step of %d streams per push, got %d steps / %d chunks"
                               % (S, b1 - b0, c1 - c0))
        res[regime] = (wall * 1000.0 / steps, toks / (steps * S), steps)
        log("%s regime: %d steps, %.4f ms/step, %.2f tokens per stream-chunk" % (regime, steps, res[regime][0],
                                                                                 res[regime][1]))
        st.close()
        dec.close()
    ms = res["blank"][0]
    value = S * T * FRAME_SEC / (ms / 1000.0)
    result = {
        "metric": "aggregate audio-sec/sec of live streaming transcription at %d streams (audio in, tokens out)" % S,
        "value": round(value, 2),
        "unit": "audio-sec/sec",
        "n_gpus": 1, "steps": res["blank"][2], "warmup": warm, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": PRECISION + " (encoder); mel frontend, joint and RNN-T fp32",
        "data": "synthetic (seeded random-init weights, harmonic test audio, Slaney-like filterbank)",
        "config": {"workload": "live streaming: %d streams x %d samples pushed per step -> mel -> subsampling -> "
                               "24 layers -> joint.enc -> greedy RNN-T, lookahead %d (%d ms chunks), every frame blank"
                               % (S, hop, la, int(T * FRAME_SEC * 1000)),
                   "streams": S, "lookahead": la, "chunk_frames": T, "layers": cfg.layers},
        "mel_us_per_step": round(mel_us, 2),
        "cap_regime_ms_per_step": round(res["cap"][0], 4),
        "cap_regime_tokens_per_stream_chunk": round(res["cap"][1], 3),
        "mixed_regime_ms_per_step": round(res["mixed"][0], 4),
        "mixed_regime_tokens_per_stream_chunk": round(res["mixed"][1], 3),
    }
    fe.close()
    enc.close()
    print(json.dumps(result), flush=True)


_LIBRARY_GEMM_SCRIPT = r"""
import json, sys, torch
M, shapes, iters = json.loads(sys.argv[1])
gen = torch.Generator(device="cuda").manual_seed(5)
out = {}
for name, (N, K) in shapes.items():
    a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=gen)
    w = torch.randn(N, K, device="cuda", dtype=torch.bfloat16, generator=gen).t().contiguous()
    for _ in range(10):
        c = torch.matmul(a, w)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        c = torch.matmul(a, w)
    e1.record()
    torch.cuda.synchronize()
    out[name] = e0.elapsed_time(e1) * 1000.0 / iters
print(json.dumps(out))
"""


def library_gemm_times(M, D, F, iters=100):
    """The vendor GEMM (torch.matmul on bf16, which runs hipBLASLt) on each projection's shape
    [M, K] x [K, N]: a reference point for the projection kernels, plain output, no fused epilogue.
    torch carries its own HIP runtime, so it runs in a child process."""
    import subprocess
    shapes = {"ff_linear1": (F, D), "ff_linear2": (D, F), "qkv": (3 * D, D), "linear_out": (D, D),
              "pointwise_conv1": (2 * D, D), "pointwise_conv2": (D, D)}
    r = subprocess.run([sys.executable, "-c", _LIBRARY_GEMM_SCRIPT, json.dumps([M, shapes, iters])],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    if r.returncode != 0:
        log("library GEMM timing failed (%d): %s" % (r.returncode, r.stderr.strip().splitlines()[-1:]))
        return None
    us = json.loads(r.stdout.strip().splitlines()[-1])
    out = {}
    for name, (N, K) in shapes.items():
        out[name] = {"us": round(us[name], 3), "tflops": round(2.0 * M * N * K / us[name] / 1e6, 1)}
        log("library GEMM %-16s %8.2f us  %7.1f TFLOP/s  (M %d, N %d, K %d)" % (name, us[name], out[name]["tflops"], M, N, K))
    return out


PRECISION = "f16 activations/K/V, bf16-valued weights, fp32 accumulation"
PRECISION_NOTE = ("16-bit encoder (UD_BF16): linear weights rounded to bf16 and held as IEEE half; activations, "
                  "K/V caches, position tables and MFMA operands IEEE half (saturating at +-65504); fp32 "
                  "accumulation, residual stream, norms and conv cache")


def projection_mfma(ud, enc, rows, mfma_f16, hs, iters=96):
    """Each projection of the step timed as the step launches it (ud_time_projection, weights from
    HBM) and the seven projections of a layer together (ff linear1/linear2 twice)."""
    per_layer = {"ff_linear1": 2, "ff_linear2": 2, "qkv": 1, "linear_out": 1, "pointwise_conv1": 1, "pointwise_conv2": 1}
    proj = {}
    tot_fl = tot_ms = 0.0
    for idx, name in enumerate(ud.Encoder.PROJECTIONS):
        pms, pfl = enc.time_projection(idx, rows, iters, hip_stream=hs)
        tf = pfl / (pms / 1000.0) / 1e12
        proj[name] = {"us": round(pms * 1000.0, 3), "tflops": round(tf, 1),
                      "frac_nominal": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "frac_measured": round(tf / mfma_f16, 4)}
        tot_fl += per_layer[name] * pfl
        tot_ms += per_layer[name] * pms
        log("projection %-16s %8.2f us  %7.1f TFLOP/s  (%d rows)" % (name, pms * 1000.0, tf, rows))
    tf = tot_fl / (tot_ms / 1000.0) / 1e12
    return {"rows": rows, "projections": proj, "layer_tflops": round(tf, 1),
            "frac_nominal": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "frac_measured": round(tf / mfma_f16, 4),
            "note": "the seven projections of a layer (ff linear1/linear2 twice), each timed as the step launches it "
                    "(ud_time_projection, weights from HBM), f16 operands with bf16-valued weights"}


def long_chunk(ud, lw, sw, args, hbm_read, mfma_f16):
    """The long-chunk workload (256 streams x 14 frames over L = 70) on one encoder with the
    default workload's weights: (1) the fused attention at that shape (the batched MFMA kernel: 103
    MB per launch, where the fixed per-launch cost is a small part), timed as the default
    workload's kernel is (HIP events over launches cycling the 24 layers' rings after one untimed
    pass); (2) the whole mel-in step (subsampling + 24 layers), steps timed back to back as the
    default workload's are; (3) its projections' MFMA use."""
    wl = WORKLOADS["chunk14"]
    S, T = wl["streams"], wl["T"]
    cfg = ud.EncoderConfig(layers=24, max_chunk=T, max_streams=S, dtype="bf16")
    L, D, H, dk = cfg.left_context, cfg.d_model, cfg.heads, cfg.d_model // cfg.heads
    enc = ud.Encoder(cfg)
    for l, w in enumerate(lw):
        enc.set_layer_weights(l, w)
    enc.set_subsampling_weights(sw)
    enc.finalize()
    streams = [enc.new_stream() for _ in range(S)]
    rng = np.random.default_rng(12)
    k = rng.standard_normal((L, D), dtype=np.float32)
    v = rng.standard_normal((L, D), dtype=np.float32)
    conv = np.zeros((cfg.conv_kernel - 1, D), np.float32)
    for i, s in enumerate(streams):           # N(0,1) rows, a different rotation per stream and layer
        for l in range(cfg.layers):
            s.import_cache(l, np.roll(k, i + 7 * l, axis=0), np.roll(v, 3 * i + 5 * l, axis=0), conv, L)
    hs = ud.HipStream()
    qkv = ud.DeviceBuffer.from_numpy(ud.f16_bits(rng.standard_normal((S * T, 3 * D), dtype=np.float32)))
    att = ud.DeviceBuffer(S * T * D * 2)
    enc.time_layer_attention(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
    ms = enc.time_layer_attention(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
    Tk, n_rel = L + T, L + 2 * T - 1
    nbytes = S * Tk * H * dk * 2 * 2 + S * 2 * T * H * dk * 2 + n_rel * H * dk * 2 + 2 * H * dk * 4
    achieved = nbytes / (ms / 1000.0) / 1e9
    log("long-chunk attention (256 streams x 14 frames): %.2f us/launch, %.0f GB/s" % (ms * 1000.0, achieved))
    roof = {"kernel": "relpos_ring_mfma_kernel (fused rel-pos attention over the K/V ring window)",
            "workload": "256 streams x 14 frames, left context 70, 8 heads x 128, %s (the long-chunk step's attention)"
                        % PRECISION,
            "us_per_launch": round(ms * 1000.0, 3), "bound": "hbm", "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "measured_peak": round(hbm_read, 1), "frac_measured": round(achieved / hbm_read, 4),
            "traffic": read_traffic("relpos_ring_chunk14"), "algorithmic_bytes_per_launch": nbytes}
    # the whole step at this shape
    rows = mel_rows(T)
    mel = ud.DeviceBuffer.from_numpy(rng.standard_normal((S, rows, 128), dtype=np.float32))
    x = ud.DeviceBuffer(S * T * D * 4)
    out = ud.DeviceBuffer(S * T * D * 4)

    def step():
        Tn, valid = enc.subsample(S, mel, x, drop=2, mel_rows=rows, hip_stream=hs)
        enc.encode_stream_step(streams, x, out, valid=valid, T=Tn, hip_stream=hs)

    warm14 = warm_up(step, hs, 10)
    n14 = 25
    e0, e1 = ud.Event(), ud.Event()
    ud.synchronize()
    e0.record(hs)
    t0 = time.perf_counter()
    for _ in range(n14):
        step()
    e1.record(hs)
    e1.synchronize()
    wall = (time.perf_counter() - t0) * 1000.0
    ms14 = max(wall, e0.elapsed_ms(e1)) / n14
    value14 = S * T * FRAME_SEC / (ms14 / 1000.0)
    log("long-chunk step (256 streams x 14 frames, 24 layers): %.4f ms/step, %.0f audio-sec/sec" % (ms14, value14))
    mf = projection_mfma(ud, enc, S * T, mfma_f16, hs, iters=24)
    flops = 2.0 * S * T * 24 * (2 * 2 * cfg.ff_dim * D + 4 * D * D + 2 * D * D + D * D)
    step_tf = flops / (ms14 / 1000.0) / 1e12
    chunk14 = {"workload": "cache-aware encoder step (dw_striding 8x subsampling + 24 layers), %d streams x %d mel "
                           "rows -> %d frames (1120 ms), left context %d, %s" % (S, rows, T, L, PRECISION),
               "ms_per_step": round(ms14, 5), "value": round(value14, 2), "unit": "audio-sec/sec",
               "steps_timed": n14, "warmup_steps": warm14, "projection_tflops_per_step": round(step_tf, 1),
               "step_frac_of_mfma_peak": round(step_tf / MFMA_BF16_PEAK_TFLOPS, 4),
               "mfma_utilisation": mf}
    enc.close()
    return roof, chunk14


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="chunk2")
    ap.add_argument("--attn-iters", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-long-chunk-attention", action="store_true",
                    help="skip the default workload's long-chunk measurements (256 streams x 14 frames: the "
                         "attention kernel, the whole step and its projections)")
    ap.add_argument("--no-other-kernels", action="store_true",
                    help="skip the default workload's offline-attention and decode-attention kernel figures")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a known-size kernel for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="chunk workloads: also time the vendor GEMM (torch.matmul, hipBLASLt) on each projection shape")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the encoder step shards by independent streams with no "
              "collective, and this build runs on a single MI355X (use --gpus 1)", file=sys.stderr)
        sys.exit(2)

    ud = load_pkg()
    if args.calibrate_copy_mib > 0:
        nbytes = args.calibrate_copy_mib << 20
        src, dst = ud.DeviceBuffer.zeros(nbytes), ud.DeviceBuffer(nbytes)
        ud.lib().ud_memcpy_dtod(dst.ptr, src.ptr, nbytes)
        ud.synchronize()
        log("calibration copy: %d MiB device-to-device" % args.calibrate_copy_mib)
        src.free(); dst.free()
    if args.workload in ("decode", "decode_mq"):
        decode_bench(ud, args, workload=args.workload)
        return
    if args.workload == "offline":
        offline_bench(ud, args)
        return
    if args.workload == "rnnt":
        rnnt_bench(ud, args)
        return
    if args.workload in ("stream", "stream14"):
        stream_bench(ud, args)
        return
    wl = WORKLOADS[args.workload]
    S, T = wl["streams"], wl["T"]
    cfg = ud.EncoderConfig(layers=24, max_chunk=T, max_streams=S, dtype="bf16")
    L, D, H, dk = cfg.left_context, cfg.d_model, cfg.heads, cfg.d_model // cfg.heads
    log("device %s; workload %s: %d streams x %d frames, L=%d, %d layers, %s"
        % (ud.device_arch(), args.workload, S, T, L, cfg.layers, PRECISION))

    lw = [ud.synthetic_layer_weights(cfg, 2024, l, ln_jitter=0.0) for l in range(cfg.layers)]
    sw = ud.synthetic_subsampling_weights(2025)
    enc = ud.Encoder(cfg)
    for l, w in enumerate(lw):
        enc.set_layer_weights(l, w)
    enc.set_subsampling_weights(sw)
    enc.finalize()
    log("weights uploaded")
    streams = [enc.new_stream() for _ in range(S)]
    rng = np.random.default_rng(11)
    conv = np.zeros((cfg.conv_kernel - 1, D), np.float32)
    for s in streams:
        for l in range(cfg.layers):
            k = rng.standard_normal((L, D), dtype=np.float32)
            v = rng.standard_normal((L, D), dtype=np.float32)
            conv[:] = rng.standard_normal(conv.shape, dtype=np.float32)
            s.import_cache(l, k, v, conv, L)
    log("caches seeded (cache_len %d)" % L)

    rows = mel_rows(T)
    mel = ud.DeviceBuffer.from_numpy(rng.standard_normal((S, rows, 128), dtype=np.float32))
    x = ud.DeviceBuffer(S * T * D * 4)
    out = ud.DeviceBuffer(S * T * D * 4)
    hs = ud.HipStream()

    def step():
        Tn, valid = enc.subsample(S, mel, x, drop=2, mel_rows=rows, hip_stream=hs)
        enc.encode_stream_step(streams, x, out, valid=valid, T=Tn, hip_stream=hs)

    for _ in range(args.warmup):
        step()
    hs.synchronize()
    log("warm-up done (%d steps)" % args.warmup)

    def timed(fn, iters):
        e0, e1 = ud.Event(), ud.Event()
        ud.synchronize()
        e0.record(hs)
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        e1.record(hs)
        e1.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1000.0
        ud.synchronize()
        return wall_ms, e0.elapsed_ms(e1)

    wall_ms, gpu_ms = timed(step, args.steps)
    ms_per_step = max(wall_ms, gpu_ms) / args.steps
    audio_per_step = S * T * FRAME_SEC
    value = audio_per_step / (ms_per_step / 1000.0)
    log("timed %d steps: %.4f ms/step (wall %.1f ms, events %.1f ms)" % (args.steps, ms_per_step, wall_ms, gpu_ms))

    # Per-step latency, as the reference reports it (p50 / p99 per step, NemotronStreamer.swift:54-64,
    # docs/PERF_LOG.md:26-28): HIP events around every step of a back-to-back run, and the host wall
    # clock of a step launched and waited for on its own.
    nlat = max(100, args.steps // 2)
    evs = [(ud.Event(), ud.Event()) for _ in range(nlat)]
    ud.synchronize()
    for a0, a1 in evs:
        a0.record(hs)
        step()
        a1.record(hs)
    hs.synchronize()
    lat = np.array([a0.elapsed_ms(a1) for a0, a1 in evs])
    sync_lat = []
    for _ in range(nlat):
        t0 = time.perf_counter()
        step()
        hs.synchronize()
        sync_lat.append((time.perf_counter() - t0) * 1000.0)
    sync_lat = np.array(sync_lat)
    pct = lambda a: {"p50": round(float(np.percentile(a, 50)), 4), "p99": round(float(np.percentile(a, 99)), 4),
                     "mean": round(float(a.mean()), 4), "max": round(float(a.max()), 4), "n": int(len(a))}
    log("step latency: events p50 %.4f p99 %.4f ms; launch+wait p50 %.4f p99 %.4f ms"
        % (np.percentile(lat, 50), np.percentile(lat, 99), np.percentile(sync_lat, 50), np.percentile(sync_lat, 99)))
    parts = max(20, args.steps // 4)
    fw, fg = timed(lambda: enc.subsample(S, mel, x, drop=2, mel_rows=rows, hip_stream=hs), parts)
    valid = np.full(S, T, np.int32)
    lw_, lg = timed(lambda: enc.encode_stream_step(streams, x, out, valid=valid, T=T, hip_stream=hs), parts)
    front_ms, layers_ms = max(fw, fg) / parts, max(lw_, lg) / parts
    log("parts: subsampling %.4f ms, 24 layers %.4f ms" % (front_ms, layers_ms))

    # Measured peaks of this device (same run), then the projections' MFMA use at this step's rows.
    hbm_read, hbm_copy = ud.measure_hbm(4 << 30, 10, hip_stream=hs)
    mfma_f16, mfma_bf16 = ud.measure_mfma(20000, hip_stream=hs)
    log("measured peaks: HBM read %.0f GB/s, copy %.0f GB/s; MFMA f16 %.0f, bf16 %.0f TFLOP/s"
        % (hbm_read, hbm_copy, mfma_f16, mfma_bf16))
    rows_step = S * T
    mfma_util = projection_mfma(ud, enc, rows_step, mfma_f16, hs)
    lib_gemm = library_gemm_times(rows_step, D, cfg.ff_dim) if args.library_gemm else None

    # The fused attention kernel alone, on the stream it is launched on.
    qkv = ud.DeviceBuffer.from_numpy(ud.f16_bits(rng.standard_normal((S * T, 3 * D), dtype=np.float32)))
    att = ud.DeviceBuffer(S * T * D * 2)
    # one untimed pass of the same loop first: the timed one then runs at steady clocks
    enc.time_layer_attention(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
    attn_ms = enc.time_layer_attention(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
    Tk, n_rel = L + T, L + 2 * T - 1
    attn_bytes = S * Tk * H * dk * 2 * 2 + S * 2 * T * H * dk * 2 + n_rel * H * dk * 2 + 2 * H * dk * 4
    achieved = attn_bytes / (attn_ms / 1000.0) / 1e9
    log("attention kernel: %.2f us/launch, %.0f GB/s" % (attn_ms * 1000.0, achieved))
    floor_ms = None
    if T <= 2:
        # the same loads with no arithmetic: what memory alone costs for this launch shape
        enc.time_ring_read_floor(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
        floor_ms = enc.time_ring_read_floor(streams, T, 0, qkv, att, args.attn_iters, hip_stream=hs)
        log("read floor of the same access pattern: %.2f us/launch, %.0f GB/s"
            % (floor_ms * 1000.0, attn_bytes / (floor_ms / 1000.0) / 1e9))

    result = {
        "metric": "aggregate audio-sec/sec at %d streams; attention-kernel %% of HBM roofline" % S,
        "value": round(value, 2),
        "unit": "audio-sec/sec",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": PRECISION,
        "precision": PRECISION_NOTE,
        "data": "synthetic (seeded random-init weights, N(0,1) inputs and caches)",
        "config": {
            "workload": "cache-aware FastConformer encoder step (dw_striding 8x subsampling + 24 layers), "
                        "%d streams x %d mel rows -> %d frames (%d ms), left context %d, %s"
                        % (S, rows, T, int(T * FRAME_SEC * 1000), L, PRECISION),
            "streams": S, "mel_rows": rows, "chunk_frames": T, "left_context": L, "layers": cfg.layers,
            "d_model": D, "heads": H, "ff_dim": cfg.ff_dim, "conv_kernel": cfg.conv_kernel,
        },
        "subsampling_ms_per_step": round(front_ms, 5),
        "layers_ms_per_step": round(layers_ms, 5),
        "step_latency_ms": dict(pct(lat), method="HIP events around each step of a back-to-back run"),
        "sync_step_latency_ms": dict(pct(sync_lat), method="host wall clock of one step launched and waited for"),
        "measured_peaks": {"hbm_read_gbs": round(hbm_read, 1), "hbm_copy_gbs": round(hbm_copy, 1),
                           "mfma_f16_tflops": round(mfma_f16, 1), "mfma_bf16_tflops": round(mfma_bf16, 1),
                           "method": "ud_measure_hbm (4 GiB buffers x 10, non-temporal streaming) and ud_measure_mfma "
                                     "(v_mfma_f32_32x32x16 register chains) in this run"},
        "mfma_utilisation": mfma_util,
        **({"library_gemm": dict(lib_gemm, method="torch.matmul bf16 (hipBLASLt) on the same [rows, K] x [K, N], "
                                               "100 back-to-back calls, HIP events; plain output, no epilogue")}
           if lib_gemm else {}),
        "realtime_factor": round(value, 2),
        "attention_steps_per_sec": round(1000.0 / attn_ms, 1),
        "attention_us_per_launch": round(attn_ms * 1000.0, 3),
        "roofline": {
            "kernel": ("relpos_ring_wave_kernel" if T <= 2 else "relpos_ring_small_kernel" if T <= 4
                       else "relpos_ring_mfma_kernel") + " (fused rel-pos attention over the K/V ring window)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "measured_peak": round(hbm_read, 1),
            "frac_measured": round(achieved / hbm_read, 4),
            "traffic": read_traffic("relpos_ring_%s" % args.workload),
            "algorithmic_bytes_per_launch": attn_bytes,
            "read_floor_us": round(floor_ms * 1000.0, 3) if floor_ms else None,
            "read_floor_frac": round(attn_bytes / (floor_ms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4) if floor_ms else None,
        },
    }
    enc.close()
    if args.workload == "chunk2" and not args.no_long_chunk_attention:
        result["roofline_long_chunk"], result["chunk14_step"] = long_chunk(ud, lw, sw, args, hbm_read, mfma_f16)
    if args.workload == "chunk2" and not args.no_other_kernels:
        result["offline_attention"] = offline_bench(ud, args, summary=True, steps=200, warmup=20)
        result["decode_attention"] = decode_bench(ud, args, summary=True, steps=200, warmup=20)
        result["decode_attention_4_queries"] = decode_bench(ud, args, summary=True, steps=200, warmup=20,
                                                            workload="decode_mq")
    if not args.no_cpu_baseline:
        cpu = host_cpu()
        # a bounded sample: all 64 streams at 2-frame chunks (about 0.7 s per step on 16 cores); at
        # 14-frame chunks the streams of about 256 rows (18 of the 256)
        S_sample = S if S * T <= 256 else max(1, 256 // T)
        log("cpu baseline: oracle on %d threads (%s), ~%.0f s" % (cpu["threads"], cpu["model"], args.cpu_seconds))
        result["cpu_baseline"] = cpu_baseline(lw, sw, cfg, S, T, args.cpu_seconds, cpu, S_sample=S_sample)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
