"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload ("C2"): Llama-3-8B-shaped decode step on one
layer — 32 query heads, 8 KV heads, head_dim 128, fp16, block_size 16, 64
sequences with context U[512,4096], block tables drawn from a randomly permuted
pool of 1.1x the needed blocks, Q/K/V = 0.3 N(0,1) (synthetic, seed 1).

One step = KV append of one token per sequence (vkv_reshape_and_cache)
followed by paged decode over ctx+1 keys (vkv_paged_decode), both through the
C ABI on torch's current stream, inputs resident in HBM.

Printed (rank 0, one JSON line): metric/value = decode KV bytes per step / step
time (GB/s); roofline = the decode operation alone (its partition and merge
kernels) timed with HIP events on the launch stream; cpu_baseline = the CPU
oracle's decode on a sample of the same sequences.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "vllm-cpp_amd", "python"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
WARM_MS = 300.0        # minimum wall time of untimed steps before the timed ones
DECODE_GROUPS, DECODE_CALLS = 11, 20


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def source_blob(rel):
    """git's blob id of a committed source file (sha1 of "blob <size>\\0" + bytes),
    computed without git, so that a summary can name the exact kernel source it
    measured and the GPU box (no .git there) can check it."""
    import hashlib
    with open(os.path.join(ROOT, rel), "rb") as f:
        data = f.read()
    return hashlib.sha1(b"blob %d\0" % len(data) + data).hexdigest()


DECODE_SRC = "vllm-cpp_amd/csrc/decode.hip"


def measured_traffic():
    """HBM bytes per decode call from the committed rocprofv3 PMC summary
    (profiles/decode_c2_traffic.json: FETCH_SIZE and WRITE_SIZE, calibrated on a
    1 GiB copy), or None with the reason when that summary is absent or was
    measured on another decode.hip than the one built here."""
    path = os.path.join(ROOT, "profiles", "decode_c2_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        traffic = int(d["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None, "no committed traffic summary"
    if d.get("decode_hip_blob") != source_blob(DECODE_SRC):
        return None, "the committed traffic summary measured another decode.hip"
    return traffic, f"profiles/decode_c2_traffic.json (commit {d.get('commit', '?')})"


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(kc, vc, q, lay, cfg, num_seqs=64, min_seconds=10.0, min_seconds_1t=8.0):
    """CPU oracle decode (oracle/kv_oracle.c, a C restatement of the reference
    kernel) on the first num_seqs sequences, repeated until min_seconds have
    passed, on the host's cores (<= 16 threads), then on one thread."""
    import numpy as np
    import torch
    from oracle import oracle
    bs = cfg.block_size
    idx = list(range(num_seqs))
    ctx = lay.context_lens[idx]
    nblk = (ctx + bs - 1) // bs
    ids = np.concatenate([lay.block_tables[s, :n] for s, n in zip(idx, nblk)])
    kk = kc[torch.from_numpy(ids).long().to(kc.device)].cpu().numpy().view(np.uint16)
    vv = vc[torch.from_numpy(ids).long().to(vc.device)].cpu().numpy().view(np.uint16)
    tables = np.zeros((num_seqs, int(nblk.max())), np.int32)
    off = 0
    for i, n in enumerate(nblk):
        tables[i, :n] = np.arange(off, off + n)
        off += int(n)
    qn = q[idx].float().cpu().numpy()
    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.paged_decode(qn[:1], kk, vv, tables[:1], np.minimum(ctx[:1], 16), cfg.scale, nthreads=1)  # tables init

    def timed(nthreads, seconds):
        reps = 0
        t0 = time.perf_counter()
        while True:
            oracle.paged_decode(qn, kk, vv, tables, ctx, cfg.scale, nthreads=nthreads)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= seconds:
                return dt, reps

    dt, reps = timed(threads, min_seconds)
    dt1, reps1 = timed(1, min_seconds_1t)
    call_bytes = int(ctx.astype(np.int64).sum()) * cfg.num_kv_heads * cfg.head_dim * 2 * 2
    return {"value": round(reps * call_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(dt / reps * 1e6, 1),
            "value_1_thread": round(reps1 * call_bytes / dt1 / 1e9, 4),
            "us_per_call_1_thread": round(dt1 / reps1 * 1e6, 1),
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": f"oracle decode (C restatement of the reference kernel) of {num_seqs} of the "
                      f"{cfg.num_seqs} C2 sequences ({int(ctx.sum())} KV tokens, fp16 KV, fp32 math): "
                      f"{reps} calls in {dt:.1f} s on {threads} threads, {reps1} calls in {dt1:.1f} s on 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10,
                    help="untimed steps before the timed ones (then more until %.0f ms have passed)" % WARM_MS)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    ap.add_argument("--partition-size", type=int, default=0,
                    help="decode split-K partition in tokens (0: the library's default)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 10 times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against a kernel of known traffic)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the paged KV path "
              "shards by sequence or KV head with no cross-GPU exchange); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] copy probe: 10 copies of 1 GiB")
        return
    cfg = workloads.config2()
    lay = cfg.layout
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    shape = (lay.num_blocks, bs, Hkv, D)
    kc = (torch.randn(shape, generator=g, device=dev) * cfg.sigma).half()
    vc = (torch.randn(shape, generator=g, device=dev) * cfg.sigma).half()
    q = (torch.randn((S, H, D), generator=g, device=dev) * cfg.sigma).half()
    nk = (torch.randn((S, Hkv, D), generator=g, device=dev) * cfg.sigma).half()
    nv = (torch.randn((S, Hkv, D), generator=g, device=dev) * cfg.sigma).half()
    slots = torch.from_numpy(lay.slots(cfg.prev_lens, np.arange(S))).to(dev)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(lay.context_lens).to(dev)
    out = torch.empty((S, H, D), dtype=torch.float16, device=dev)
    P = args.partition_size
    ws = torch.zeros(vkv.decode_workspace_size(out, q, kc, vc, bt, cl, cfg.scale, partition_size=P) // 4 + 4,
                     dtype=torch.float32, device=dev)  # first 256 bytes: counters, zero before first use
    stream = torch.cuda.current_stream()

    def append():
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, stream=stream)

    def decode():
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, workspace=ws, stream=stream, partition_size=P)

    def step():
        # one decode step of the attention layer: the append of each
        # sequence's new token fused into the decode launches
        vkv.paged_decode_append(out, q, kc, vc, bt, cl, cfg.scale, nk, nv, slots, workspace=ws, stream=stream,
                                partition_size=P)

    def step_two_calls():
        append()
        decode()

    def timed(fn, n):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    # `warmup` steps, then more until WARM_MS of wall time has passed: an idle
    # GPU's clocks take ~0.2 s to rise, and a run warmed by 5 steps alone timed
    # the decode ~4 % slow.
    t_w = time.perf_counter()
    warm_steps = _warm(step, args.warmup, min_ms=WARM_MS)
    warm_ms = (time.perf_counter() - t_w) * 1e3
    log(f"[bench] warmup done: {warm_steps} steps in {warm_ms:.0f} ms ({args.warmup} asked), pool "
        f"{lay.num_blocks} blocks ({2 * kc.numel() * 2 / 1e9:.2f} GB K+V)")
    ms_step = timed(step, args.steps)
    log(f"[bench] timed {args.steps} steps: {ms_step * 1e3:.1f} us/step")
    _warm(step_two_calls, 0, min_ms=50.0)
    ms_step2 = timed(step_two_calls, args.steps)
    log(f"[bench] the same steps as two calls (append, then decode): {ms_step2 * 1e3:.1f} us/step")
    # the decode call alone: median, p10 and p90 over DECODE_GROUPS samples,
    # each the mean of DECODE_CALLS back-to-back calls
    dec = _events_ms(decode, DECODE_GROUPS * DECODE_CALLS, stream, groups=DECODE_GROUPS)
    ms_decode = dec[0]
    ms_append = _events_ms(append, DECODE_GROUPS * DECODE_CALLS, stream, groups=DECODE_GROUPS)[0]
    log(f"[bench] decode {ms_decode * 1e3:.1f} us (p10 {dec[1] * 1e3:.1f}, p90 {dec[2] * 1e3:.1f}), "
        f"append {ms_append * 1e3:.1f} us")

    # the box's read-only ceiling for this byte set: whole blocks of the
    # decode's block tables gathered with no math
    try:
        nblk = (lay.context_lens.astype(np.int64) + bs - 1) // bs
        ids = np.concatenate([lay.block_tables[s, :n] for s, n in enumerate(nblk)]).astype(np.int32)
        ceil_gbs, ceil_shape, ceil_bytes = gather_ceiling(dev, kc, vc, ids, bs * Hkv * D * 2, stream)
        ceiling = {"gbs": round(ceil_gbs, 1), "bytes": ceil_bytes, "shape": ceil_shape,
                   "workload": f"read-only gather of the {ids.shape[0]} K and V blocks ({bs * Hkv * D * 2} B each) "
                               "of the decode's block tables, no math (vllm-cpp_amd/bench/ceilings.hip)"}
        log(f"[bench] read-only gather ceiling {ceil_gbs:.0f} GB/s ({ceil_shape})")
    except RuntimeError as e:
        ceiling = {"gbs": None, "error": str(e)}

    kv_bytes = cfg.kv_bytes(2)
    traffic, traffic_note = measured_traffic()
    value = kv_bytes / (ms_step * 1e-3) / 1e9
    achieved = kv_bytes / (ms_decode * 1e-3) / 1e9
    append_bytes = S * Hkv * D * 2 * 2 * 2 + S * 4
    result = {
        "metric": "paged-decode KV GB/s (% of HBM peak) @Llama-3-8B shape; decode tokens/s/GPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "C2: Llama-3-8B-shaped paged decode, one layer, H32/Hkv8/D128 fp16, bs16, "
                               "B=64, ctx U[512,4096], append 1 token + decode per step "
                               "(vkv_paged_decode_append: the append fused into the decode launches)",
                   "global_batch": S, "context_tokens": int(lay.context_lens.sum()), "seed": cfg.seed},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "decode_tokens_per_s": round(S / (ms_step * 1e-3), 1),
        "decode_tokens_per_s_32_layers": round(S / (32 * ms_step * 1e-3), 1),
        "decode_us": round(ms_decode * 1e3, 2),
        "decode_us_p10_p90": [round(dec[1] * 1e3, 2), round(dec[2] * 1e3, 2)],
        "decode_timing": f"median of {DECODE_GROUPS} samples, each the mean of {DECODE_CALLS} back-to-back "
                         "calls timed with HIP events on the launch stream",
        "warm_steps": warm_steps,
        "warm_ms": round(warm_ms, 1),
        "step_us_two_calls": round(ms_step2 * 1e3, 2),
        "step_two_calls_note": "the same step as vkv_reshape_and_cache then vkv_paged_decode (the reference's "
                               "call pattern), timed after the headline steps",
        "append_us": round(ms_append * 1e3, 2),
        "append_gbs": round(append_bytes / (ms_append * 1e-3) / 1e9, 2),
        "kv_bytes_per_call": kv_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_over_algorithmic": None if traffic is None else round(traffic / kv_bytes, 4),
                     "traffic_source": traffic_note,
                     "kernel": "paged decode (partition + merge kernels), event-timed on the launch stream",
                     "achieved_note": "algorithmic KV bytes per call / decode call time",
                     "measured_ceiling": ceiling["gbs"],
                     "frac_of_measured_ceiling": None if not ceiling["gbs"] else round(achieved / ceiling["gbs"], 4)},
        "hbm_read_ceiling": ceiling,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(kc, vc, q, lay, cfg)
        log(f"[bench] cpu baseline: {result['cpu_baseline']['sample']}")
    print(json.dumps(result), flush=True)


# --------------------------------------------------------------------------
# --suite: the other rows of the path, one JSON line each (not the headline).


def _warm(fn, warmup, min_ms=200.0):
    """`warmup` untimed calls, then more until min_ms of wall time has passed:
    an idle GPU's clocks take a while to rise, and a short kernel timed right
    away runs slow."""
    import torch
    n = 0
    for _ in range(warmup):
        fn()
        n += 1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
    return n


def _events_ms(fn, n, stream, groups=5):
    """Median, p10 and p90 over `groups` samples of the mean time of n
    back-to-back calls (HIP events on the launch stream), in ms."""
    import numpy as np
    import torch
    n = max(1, n // groups)
    v = []
    for _ in range(groups):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        v.append(e0.elapsed_time(e1) / n)
    v = np.array(v)
    return float(np.median(v)), float(np.percentile(v, 10)), float(np.percentile(v, 90))


def _cpu_time(fn, min_seconds=3.0):
    """Seconds per call of a CPU oracle function, repeated for >= min_seconds."""
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            return dt / reps, reps


def _cpu_threads():
    return max(1, min(16, os.cpu_count() or 1))


def _rand_half(shape, g, dev, sigma):
    import torch
    return (torch.randn(shape, generator=g, device=dev) * sigma).half()


def suite_c3(dev, steps, warmup):
    """C3 mixed step: append of the step's 4216 tokens, then one paged_prefill call over
    8 prefill chunks (512 tokens on prior U[0,2048]) and 120 decodes (ctx U[1024,8192])."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config3()
    lay = cfg.layout
    H, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    g = torch.Generator(device=dev).manual_seed(2)
    kc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    vc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    qsl_np = cfg.query_start_loc
    Tq = int(qsl_np[-1])
    q = _rand_half((Tq, H, D), g, dev, 0.3)
    nk = _rand_half((Tq, Hkv, D), g, dev, 0.3)
    nv = _rand_half((Tq, Hkv, D), g, dev, 0.3)
    seqs = np.repeat(np.arange(len(cfg.q_lens)), cfg.q_lens)
    pos = np.concatenate([np.arange(p, p + n) for p, n in zip(cfg.prior_lens, cfg.q_lens)])
    slots = torch.from_numpy(lay.slots(pos, seqs)).to(dev)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(lay.context_lens).to(dev)
    qsl = torch.from_numpy(qsl_np).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    mql = int(cfg.q_lens.max())

    def append():
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, stream=stream)

    # the host-built work list of the prefill rows (an engine builds it once
    # per step beside its other metadata, for every layer)
    wl = torch.from_numpy(vkv.prefill_work_list(out, q, kc, vc, bt, cl, qsl, mql, cfg.scale, qsl_np,
                                                lay.context_lens)).to(dev)

    def attn():
        vkv.paged_prefill(out, q, kc, vc, bt, cl, qsl, mql, cfg.scale, stream=stream, work_list=wl)

    def attn_unlisted():
        vkv.paged_prefill(out, q, kc, vc, bt, cl, qsl, mql, cfg.scale, stream=stream)

    _warm(lambda: (append(), attn(), attn_unlisted()), warmup)
    torch.cuda.synchronize()
    t_app = _events_ms(append, steps, stream)
    # the two variants alternate, three rounds each (the call's time drifts
    # with the clocks by more than their difference); the round with the
    # median time is reported
    rounds = sorted((_events_ms(attn, steps, stream), _events_ms(attn_unlisted, steps, stream)) for _ in range(3))
    t_att = sorted(r[0] for r in rounds)[1]
    t_un = sorted(r[1] for r in rounds)[1]
    npf = int((cfg.q_lens > 1).sum())
    # attended keys per prefill query row: prior + j + 1; FLOPs = 4 D per (query head, key)
    keys = sum(int(cfg.prior_lens[s]) * int(cfg.q_lens[s]) + int(cfg.q_lens[s]) * (int(cfg.q_lens[s]) + 1) // 2
               for s in range(npf))
    flops = 4.0 * D * H * keys
    dec_bytes = int(lay.context_lens[npf:].astype(np.int64).sum()) * Hkv * D * 2 * 2
    return {"row": "C3 mixed prefill+decode", "workload": "Qwen2.5-7B shape H28/Hkv4/D128 fp16 bs32; "
            "8 x 512-token chunks on prior U[0,2048] + 120 decodes ctx U[1024,8192]; seed 2",
            "query_tokens": Tq, "append_us_median": round(t_app[0] * 1e3, 2),
            "prefill_call_us_median": round(t_att[0] * 1e3, 2), "prefill_call_us_p10_p90":
            [round(t_att[1] * 1e3, 2), round(t_att[2] * 1e3, 2)],
            "work_list": "host-built (vkv_prefill_work_list_host), built once before the timed calls",
            "prefill_call_us_in_kernel_list": round(t_un[0] * 1e3, 2),
            "prefill_rows_gflop": round(flops / 1e9, 2), "decode_rows_kv_bytes": dec_bytes,
            "step_us": round((t_app[0] + t_att[0]) * 1e3, 2)}


def suite_c3_prefill_only(dev, steps, warmup):
    """The 8 prefill sequences of C3 alone (matrix-core kernel only): TFLOP/s."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config3()
    lay = cfg.layout
    H, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    npf = int((cfg.q_lens > 1).sum())
    g = torch.Generator(device=dev).manual_seed(2)
    kc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    vc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    ql = cfg.q_lens[:npf]
    qsl_np = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    Tq = int(qsl_np[-1])
    q = _rand_half((Tq, H, D), g, dev, 0.3)
    bt = torch.from_numpy(np.ascontiguousarray(lay.block_tables[:npf])).to(dev)
    cl = torch.from_numpy(np.ascontiguousarray(lay.context_lens[:npf])).to(dev)
    qsl = torch.from_numpy(qsl_np).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def attn():
        vkv.paged_prefill(out, q, kc, vc, bt, cl, qsl, int(ql.max()), cfg.scale, stream=stream,
                          multi_token_only=True)

    _warm(attn, warmup)
    t_kernel_list = _events_ms(attn, steps, stream)
    # the same call with the host-built work list (an engine builds it once per
    # step beside its other metadata, for every layer): the headline of the row
    words = vkv.prefill_work_list(out, q, kc, vc, bt, cl, qsl, int(ql.max()), cfg.scale, qsl_np,
                                  lay.context_lens[:npf])
    wl = torch.from_numpy(words).to(dev)

    def attn_listed():
        vkv.paged_prefill(out, q, kc, vc, bt, cl, qsl, int(ql.max()), cfg.scale, stream=stream,
                          multi_token_only=True, work_list=wl)

    _warm(attn_listed, warmup)
    t = _events_ms(attn_listed, steps, stream)
    keys = sum(int(cfg.prior_lens[s]) * int(ql[s]) + int(ql[s]) * (int(ql[s]) + 1) // 2 for s in range(npf))
    flops = 4.0 * D * H * keys
    tf = flops / (t[0] * 1e-3) / 1e12
    # the same sequences over an FP8 cache (the pool quantised by the FP8 append)
    k8 = torch.empty((lay.num_blocks, bs, Hkv, D), dtype=torch.uint8, device=dev)
    v8 = torch.empty_like(k8)
    ks8 = torch.empty((lay.num_blocks, bs, Hkv), dtype=torch.float32, device=dev)
    vs8 = torch.empty_like(ks8)
    all_slots = torch.arange(lay.num_blocks * bs, dtype=torch.int32, device=dev)
    vkv.reshape_and_cache(kc.reshape(-1, Hkv, D), vc.reshape(-1, Hkv, D), k8, v8, all_slots, ks8, vs8)

    wl8 = torch.from_numpy(vkv.prefill_work_list(out, q, k8, v8, bt, cl, qsl, int(ql.max()), cfg.scale, qsl_np,
                                                 lay.context_lens[:npf], key_scales=ks8, value_scales=vs8)).to(dev)

    def attn8():
        vkv.paged_prefill(out, q, k8, v8, bt, cl, qsl, int(ql.max()), cfg.scale, key_scales=ks8, value_scales=vs8,
                          stream=stream, multi_token_only=True, work_list=wl8)

    _warm(attn8, warmup)
    t8 = _events_ms(attn8, steps, stream)
    tf8 = flops / (t8[0] * 1e-3) / 1e12
    # CPU: the oracle's prefill (one decode per query row, as the reference) of sequence 0
    from oracle import oracle
    n0 = int(lay.context_lens[0])
    nb0 = (n0 + bs - 1) // bs
    ids = torch.from_numpy(lay.block_tables[0, :nb0]).long().to(dev)
    hk = kc[ids].cpu().numpy().view(np.uint16)
    hv = vc[ids].cpu().numpy().view(np.uint16)
    hq = q[:int(ql[0])].float().cpu().numpy()
    thr = _cpu_threads()
    fn_cpu = lambda: oracle.paged_prefill(hq, hk, hv, np.arange(nb0, dtype=np.int32)[None, :],
                                          np.array([n0], np.int32), np.array([0, int(ql[0])], np.int32),
                                          cfg.scale, nthreads=thr)
    sec, reps = _cpu_time(fn_cpu)
    keys0 = int(cfg.prior_lens[0]) * int(ql[0]) + int(ql[0]) * (int(ql[0]) + 1) // 2
    return {"row": "C3 prefill sequences alone", "workload": "the 8 x 512-token chunks of C3 (prior U[0,2048]), "
                                                          "one vkv_paged_prefill call with multi_token_only = 1",
            "us_median": round(t[0] * 1e3, 2), "us_p10_p90": [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)],
            "work_list": "host-built (vkv_prefill_work_list_host), built once before the timed calls",
            "us_median_in_kernel_list": round(t_kernel_list[0] * 1e3, 2),
            "gflop": round(flops / 1e9, 2), "tflops": round(tf, 1),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": round(tf / 2500.0, 4)},
            "fp8_cache": {"us_median": round(t8[0] * 1e3, 2), "tflops": round(tf8, 1),
                          "frac_of_fp16_peak": round(tf8 / 2500.0, 4),
                          "note": "FP8 e4m3 codes + per-(token, head) scales, dequantised to fp16 for the fp16 MFMAs"},
            "cpu_baseline": {"tflops": round(4.0 * D * H * keys0 / sec / 1e12, 5), "cores": thr, "kind": "port",
                             "sample": f"oracle prefill (one decode per query row) of sequence 0 "
                                       f"({int(ql[0])} queries on {n0 - int(ql[0])} prior keys), {reps} calls"}}


def suite_c1(dev, steps, warmup):
    """C1 (Qwen2.5-0.5B layer, 4 sequences): append + decode; launch-bound at this size."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config1()
    lay = cfg.layout
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    g = torch.Generator(device=dev).manual_seed(0)
    kc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, cfg.sigma)
    vc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, cfg.sigma)
    q = _rand_half((S, H, D), g, dev, cfg.sigma)
    nk = _rand_half((S, Hkv, D), g, dev, cfg.sigma)
    nv = _rand_half((S, Hkv, D), g, dev, cfg.sigma)
    slots = torch.from_numpy(lay.slots(cfg.prev_lens, np.arange(S))).to(dev)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(lay.context_lens).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def step():
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, stream=stream)
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=stream)

    def fused_step():
        vkv.paged_decode_append(out, q, kc, vc, bt, cl, cfg.scale, nk, nv, slots, stream=stream)

    _warm(step, warmup)
    t = _events_ms(step, steps, stream)
    _warm(fused_step, warmup)
    tf = _events_ms(fused_step, steps, stream)
    kvb = cfg.kv_bytes(2)
    # The same step captured once in a HIP graph and replayed (the launch-bound
    # case graphs are for): the capture stream's library workspace is sized by
    # an eager call on it first (a workspace cannot grow under capture).
    ref_out = out.clone()
    cs = torch.cuda.Stream()
    cs.wait_stream(stream)
    with torch.cuda.stream(cs):
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, stream=cs)
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=cs)
    cs.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, stream=cs)
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=cs)
    out.fill_(float("nan"))
    _warm(graph.replay, warmup)
    tg = _events_ms(graph.replay, steps, stream)
    graph_equal = bool(torch.equal(out.view(torch.int16), ref_out.view(torch.int16)))
    native = _native_c1(vkv, nk, nv, kc, vc, slots, out, q, bt, cl, cfg.scale, stream, steps, warmup)
    from oracle import oracle
    hk, hv = kc.cpu().numpy().view(np.uint16), vc.cpu().numpy().view(np.uint16)
    hnk, hnv = nk.cpu().numpy().view(np.uint16), nv.cpu().numpy().view(np.uint16)
    hq = q.float().cpu().numpy()
    hs = slots.cpu().numpy()

    def cpu_step():
        oracle.reshape_and_cache(hnk, hnv, hk, hv, hs)
        oracle.paged_decode(hq, hk, hv, lay.block_tables, lay.context_lens, cfg.scale, nthreads=1)

    sec, reps = _cpu_time(cpu_step)
    return {"row": "C1 append + decode", "workload": "Qwen2.5-0.5B shape H14/Hkv2/D64 fp16 bs16, B=4, ctx U[1,512]",
            "kv_bytes": kvb, "step_us_median": round(t[0] * 1e3, 2),
            "step_us_p10_p90": [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)],
            "fused_step_us_median": round(tf[0] * 1e3, 2),
            "fused_step_us_p10_p90": [round(tf[1] * 1e3, 2), round(tf[2] * 1e3, 2)],
            "note": "launch-bound: three kernels (append, partition, merge) for 0.6 MB of KV; "
                    "vkv_paged_decode_append fuses the append into the decode's two",
            "graph_step_us_median": round(tg[0] * 1e3, 2), "graph_output_equals_eager": graph_equal,
            "native_caller": native,
            "cpu_baseline": {"us_per_step": round(sec * 1e6, 1), "cores": 1, "kind": "port",
                             "sample": f"oracle append + decode of the whole step, {reps} steps"}}


STEPLOOP_LIB = os.path.join(ROOT, "vllm-cpp_amd", "lib", "libvkv_steploop.so")


def _native_c1(vkv, nk, nv, kc, vc, slots, out, q, bt, cl, scale, stream, steps, warmup):
    """The same C1 step from a native caller (vllm-cpp_amd/bench/step_loop.cpp):
    parameter structs built once, the loop in C, eager and as a replayed
    one-step HIP graph; event-timed on the launch stream."""
    import ctypes
    if not os.path.exists(STEPLOOP_LIB):
        raise RuntimeError(f"{STEPLOOP_LIB} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(STEPLOOP_LIB)
    vp = ctypes.c_void_p
    lib.vkvb_step_loop.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
    lib.vkvb_graph_create.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(vp)]
    lib.vkvb_graph_launch.argtypes = [vp, ctypes.c_int, vp]
    lib.vkvb_graph_destroy.argtypes = [vp]
    ap = vkv.append_params(nk, nv, kc, vc, slots)
    dp = vkv.decode_params(out, q, kc, vc, bt, cl, scale)
    h = stream.cuda_stream
    n = max(steps, 100)
    res = {"sample": f"5 samples of {n} back-to-back steps each"}
    for fused, tag in ((0, "two_calls"), (1, "fused")):
        def eager():
            _ck(lib.vkvb_step_loop(ctypes.byref(ap), ctypes.byref(dp), n, fused, h), "vkvb_step_loop")

        _warm(eager, warmup, min_ms=100.0)
        t = _events_ms(eager, 5, stream, groups=5)
        g = vp()
        _ck(lib.vkvb_graph_create(ctypes.byref(ap), ctypes.byref(dp), fused, ctypes.byref(g)), "vkvb_graph_create")
        try:
            def replay():
                _ck(lib.vkvb_graph_launch(g, n, h), "vkvb_graph_launch")
            _warm(replay, warmup, min_ms=100.0)
            tg = _events_ms(replay, 5, stream, groups=5)
        finally:
            lib.vkvb_graph_destroy(g)
        res[tag] = {"eager_step_us_median": round(t[0] * 1e3 / n, 2),
                    "eager_step_us_p10_p90": [round(t[1] * 1e3 / n, 2), round(t[2] * 1e3 / n, 2)],
                    "graph_step_us_median": round(tg[0] * 1e3 / n, 2)}
    return res


def suite_c5(dev, steps, warmup):
    """C5: FP8 (e4m3fn + per-token scales) append of 256 tokens and decode over
    lognormal contexts (B=256, E[ctx] ~ 3.3k)."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config5()
    lay = cfg.layout
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    g = torch.Generator(device=dev).manual_seed(4)
    N = lay.num_blocks
    kc = torch.empty((N, bs, Hkv, D), dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((N, bs, Hkv), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    all_slots = torch.arange(N * bs, dtype=torch.int32, device=dev)
    chunk = 1 << 20
    for s0 in range(0, N * bs, chunk):  # fill the pool through the FP8 append: N(0,1), 1 % outliers x8
        n = min(chunk, N * bs - s0)
        x = torch.randn((2, n, Hkv, D), generator=g, device=dev)
        x = torch.where(torch.rand(x.shape, generator=g, device=dev) < 0.01, x * 8, x).half()
        vkv.reshape_and_cache(x[0], x[1], kc, vc, all_slots[s0:s0 + n], ks, vs)
        del x
    q = _rand_half((S, H, D), g, dev, 1.0)
    nk = _rand_half((S, Hkv, D), g, dev, 1.0)
    nv = _rand_half((S, Hkv, D), g, dev, 1.0)
    slots = torch.from_numpy(lay.slots(cfg.prev_lens, np.arange(S))).to(dev)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(lay.context_lens).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def append():
        vkv.reshape_and_cache(nk, nv, kc, vc, slots, ks, vs, stream=stream)

    def decode():
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, key_scales=ks, value_scales=vs, stream=stream)

    _warm(lambda: (append(), decode()), warmup)
    torch.cuda.synchronize()
    ta = _events_ms(append, steps, stream)
    # the decode as the headline times C2's: warmed by time, then the median of
    # DECODE_GROUPS samples of DECODE_CALLS back-to-back calls
    _warm(decode, warmup, min_ms=WARM_MS)
    td = _events_ms(decode, DECODE_GROUPS * DECODE_CALLS, stream, groups=DECODE_GROUPS)
    kvb = cfg.kv_bytes(1, 4)
    gbs = kvb / (td[0] * 1e-3) / 1e9
    from oracle import oracle
    idx = list(range(16))
    ctx = lay.context_lens[idx]
    nblk = (ctx + bs - 1) // bs
    ids_np = np.concatenate([lay.block_tables[s_, :n_] for s_, n_ in zip(idx, nblk)])
    ids = torch.from_numpy(ids_np).long().to(dev)
    hk, hv = kc[ids].cpu().numpy(), vc[ids].cpu().numpy()
    hks, hvs = ks[ids].cpu().numpy(), vs[ids].cpu().numpy()
    tabs = np.zeros((16, int(nblk.max())), np.int32)
    off = 0
    for i_, n_ in enumerate(nblk):
        tabs[i_, :n_] = np.arange(off, off + n_)
        off += int(n_)
    hq = q[idx].float().cpu().numpy()
    thr = _cpu_threads()
    sec, reps = _cpu_time(lambda: oracle.paged_decode(hq, hk, hv, tabs, ctx, cfg.scale, key_scales=hks,
                                                      value_scales=hvs, nthreads=thr))
    cpu_bytes = int(ctx.astype(np.int64).sum()) * Hkv * (2 * D + 8)
    return {"row": "C5 FP8 append + decode", "workload": "H32/Hkv8/D128, bs16, B=256, ctx = clip(lognormal(7.6,1),128,32768)",
            "context_tokens": int(lay.context_lens.astype(np.int64).sum()), "kv_bytes": kvb,
            "decode_us_median": round(td[0] * 1e3, 2), "decode_us_p10_p90": [round(td[1] * 1e3, 2), round(td[2] * 1e3, 2)],
            "append_us_median": round(ta[0] * 1e3, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "cpu_baseline": {"gbs": round(cpu_bytes / sec / 1e9, 3), "cores": thr, "kind": "port",
                             "sample": f"oracle FP8 decode of sequences 0-15 ({int(ctx.sum())} tokens), {reps} calls"}}


def suite_append(dev, steps, warmup):
    """reshape_and_cache T-sweep at the C2 shape (Hkv8, D128, bs16): fp16 -> fp16 and
    fp16 -> FP8 (+ scales), slots a random permutation of a 1.25x pool."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    Hkv, D, bs = 8, 128, 16
    rows = []
    stream = torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(5)
    for T in (4216, 65536, 262144):
        N = (int(T * 1.25) + bs - 1) // bs
        perm = torch.randperm(N * bs, generator=torch.Generator().manual_seed(T))[:T].int().to(dev)
        k = _rand_half((T, Hkv, D), g, dev, 0.3)
        v = _rand_half((T, Hkv, D), g, dev, 0.3)
        for kind in ("f16", "fp8"):
            if kind == "f16":
                kc = torch.zeros((N, bs, Hkv, D), dtype=torch.float16, device=dev)
                vc = torch.zeros_like(kc)
                ks = vs = None
                wbytes = T * Hkv * D * 2 * 2
            else:
                kc = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=dev)
                vc = torch.zeros_like(kc)
                ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=dev)
                vs = torch.zeros_like(ks)
                wbytes = T * Hkv * (D + 4) * 2

            def fn():
                vkv.reshape_and_cache(k, v, kc, vc, perm, ks, vs, stream=stream)

            _warm(fn, warmup)
            t = _events_ms(fn, steps, stream)
            nbytes = T * Hkv * D * 2 * 2 + wbytes + T * 4
            gbs = nbytes / (t[0] * 1e-3) / 1e9
            row = {"tokens": T, "cache": kind, "us_median": round(t[0] * 1e3, 2), "bytes": nbytes,
                   "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
            if T == 65536:
                from oracle import oracle
                # the FP8 oracle encodes by brute force (nearest of 127 magnitudes): time a
                # 4096-token slice of the same workload for it
                Tc = T if kind == "f16" else 4096
                hk = k[:Tc].cpu().numpy().view(np.uint16)
                hv = v[:Tc].cpu().numpy().view(np.uint16)
                hp = perm[:Tc].cpu().numpy()
                cpu_bytes = nbytes * Tc // T
                if kind == "f16":
                    hkc = np.zeros((N, bs, Hkv, D), np.uint16)
                    hvc = np.zeros_like(hkc)
                    fn_cpu = lambda: oracle.reshape_and_cache(hk, hv, hkc, hvc, hp)
                else:
                    hkc = np.zeros((N, bs, Hkv, D), np.uint8)
                    hvc = np.zeros_like(hkc)
                    hks = np.zeros((N, bs, Hkv), np.float32)
                    hvs = np.zeros_like(hks)
                    fn_cpu = lambda: oracle.reshape_and_cache(hk, hv, hkc, hvc, hp, hks, hvs)
                sec, reps = _cpu_time(fn_cpu)
                row["cpu_baseline"] = {"gbs": round(cpu_bytes / sec / 1e9, 3), "cores": 1, "kind": "port",
                                       "sample": f"oracle append (the reference's per-token row copy) of the first "
                                                 f"{Tc} of the same {T} tokens, {reps} calls"}
            rows.append(row)
            del kc, vc, ks, vs
        del k, v
        torch.cuda.empty_cache()
    return {"row": "append (reshape_and_cache) T-sweep", "workload": "Hkv8/D128 fp16 source, bs16, random slots",
            "sweep": rows, "roofline_bound": "hbm", "peak": HBM_PEAK_GBS}


def suite_rope(dev, steps, warmup):
    """Fused RoPE + append (vkv_rope_reshape_and_cache) at the C2 head shape (H32/Hkv8/D128
    fp16, bs16), fp16 and FP8 caches, T in {64 (C2's step), 4216, 65536}; beside it the
    unfused pair (rope in place, then reshape_and_cache) on the same inputs."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    H, Hkv, D, bs, P = 32, 8, 128, 16, 8192
    cs = torch.from_numpy(vkv.rope_cos_sin_host(500000.0, D, P)).to(dev)
    stream = torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(6)
    rows = []
    for T in (64, 4216, 65536):
        N = (int(T * 1.25) + bs - 1) // bs
        perm = torch.randperm(N * bs, generator=torch.Generator().manual_seed(T))[:T].int().to(dev)
        pos = torch.randint(0, P, (T,), generator=torch.Generator().manual_seed(T + 1)).int().to(dev)
        q = _rand_half((T, H, D), g, dev, 0.3)
        k = _rand_half((T, Hkv, D), g, dev, 0.3)
        v = _rand_half((T, Hkv, D), g, dev, 0.3)
        for kind in ("f16", "fp8"):
            cdt = torch.float16 if kind == "f16" else torch.uint8
            kc = torch.zeros((N, bs, Hkv, D), dtype=cdt, device=dev)
            vc = torch.zeros_like(kc)
            ks = vs = None
            if kind == "fp8":
                ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=dev)
                vs = torch.zeros_like(ks)

            def fused():
                vkv.rope_reshape_and_cache(q, k, v, cs, positions=pos, key_cache=kc, value_cache=vc,
                                           slot_mapping=perm, key_scales=ks, value_scales=vs, stream=stream)

            def unfused():
                vkv.rope_reshape_and_cache(q, k, None, cs, positions=pos, stream=stream)
                vkv.reshape_and_cache(k, v, kc, vc, perm, ks, vs, stream=stream)

            _warm(lambda: (fused(), unfused()), warmup)
            torch.cuda.synchronize()
            tf = _events_ms(fused, steps, stream)
            tu = _events_ms(unfused, steps, stream)
            ceb = 2 if kind == "f16" else 1
            nbytes = (T * H * D * 2 * 2 + T * Hkv * D * 2 * 2 + T * Hkv * (D * ceb + (4 if kind == "fp8" else 0)) * 2
                      + T * D * 4 + T * 8)
            gbs = nbytes / (tf[0] * 1e-3) / 1e9
            rows.append({"tokens": T, "cache": kind, "fused_us": round(tf[0] * 1e3, 2),
                         "unfused_us": round(tu[0] * 1e3, 2), "bytes": nbytes, "gbs": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del kc, vc, ks, vs
        del q, k, v
        torch.cuda.empty_cache()
    return {"row": "fused RoPE + append", "workload": "H32/Hkv8/D128 fp16 q/k/v, bs16, random slots and positions",
            "sweep": rows, "roofline_bound": "hbm", "peak": HBM_PEAK_GBS,
            "bytes_counted": "q read+write, k and v read, cache rows (+ FP8 scales) written, one table row "
                             "(D fp32) and slot + position per token"}


def suite_step(dev, steps, warmup):
    """Batched attention step (AttentionMetadata + PagedAttentionLayer, 32 layers of
    Llama-3-8B attention, C2's 64 sequences) beside the reference's per-sequence,
    per-token call pattern on the same kernels: vllm-cpp_amd/_build/bench_attention_step."""
    import subprocess
    exe = os.path.join(ROOT, "vllm-cpp_amd", "_build", "bench_attention_step")
    if not os.path.exists(exe):
        raise RuntimeError(f"{exe} not built: run __graft_entry__.build()")
    r = subprocess.run([exe, "32", str(max(5, steps // 5)), "2"], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"bench_attention_step failed ({r.returncode}): {r.stdout[-2000:]} {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def suite_stream(dev, steps, warmup):
    """Device-to-device copy of 1 GiB (read + write): the practical HBM ceiling."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    _warm(lambda: dst.copy_(src), warmup)
    t = _events_ms(lambda: dst.copy_(src), steps, stream)
    gbs = 2 * (1 << 30) / (t[0] * 1e-3) / 1e9
    return {"row": "copy ceiling", "workload": "torch copy_ of 1 GiB on the device", "us_median": round(t[0] * 1e3, 1),
            "gbs_read_plus_write": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


CEIL_LIB = os.path.join(ROOT, "vllm-cpp_amd", "lib", "libvkv_ceilings.so")
MFMA_PEAK_TFLOPS = 2500.0  # MI355X published dense fp16 MFMA rate
HOST_LINK_GBS = 64.0       # PCIe 5.0 x16, one direction


def _ceil_lib():
    """The measurement-only kernels of vllm-cpp_amd/bench/ceilings.hip."""
    import ctypes
    if not os.path.exists(CEIL_LIB):
        raise RuntimeError(f"{CEIL_LIB} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(CEIL_LIB)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    sig = {"vkvc_mfma_loop": [vp, i32, i32, vp],
           "vkvc_read_stream": [vp, i64, vp, i32, i32, vp],
           "vkvc_read_blocks": [vp, vp, vp, i32, i64, vp, i32, i32, vp],
           "vkvc_read_heads": [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp],
           "vkvc_copy": [vp, vp, i64, vp]}
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, i32
    return lib


def _ck(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} returned {rc}")


def _cus(dev):
    import torch
    return torch.cuda.get_device_properties(dev).multi_processor_count


def gather_ceiling(dev, k_pool, v_pool, ids, block_bytes, stream, calls=20):
    """Read-only gather of whole blocks `ids` (int32 numpy) from the K and V
    pools with no math: the best over launch shapes and load kinds of the
    median of 5 samples, each the mean of calls/5 launches.  Returns
    (GB/s, shape note, bytes per launch)."""
    import torch
    lib = _ceil_lib()
    d_ids = torch.from_numpy(ids.astype("int32")).to(dev)
    cus = _cus(dev)
    out = torch.empty(cus * 8 * 256, dtype=torch.int32, device=dev)
    h = stream.cuda_stream
    nbytes = 2 * int(ids.shape[0]) * block_bytes
    best = (0.0, "")
    for mult in (2, 4, 8):
        for nt in (0, 1):
            def run():
                _ck(lib.vkvc_read_blocks(k_pool.data_ptr(), v_pool.data_ptr(), d_ids.data_ptr(), int(ids.shape[0]),
                                         block_bytes, out.data_ptr(), cus * mult, nt, h), "vkvc_read_blocks")
            _warm(run, 3, min_ms=20.0)
            t = _events_ms(run, calls, stream)
            gbs = nbytes / (t[0] * 1e-3) / 1e9
            if gbs > best[0]:
                best = (gbs, f"{cus * mult} workgroups, {'non-temporal' if nt else 'ordinary'} loads")
    return best[0], best[1], nbytes


def suite_ceilings(dev, steps, warmup):
    """Measured ceilings: dense v_mfma_f32_16x16x32_f16, read-only HBM stream
    (4 GiB), read-only block gathers of C2 and C5 (the decode's byte sets),
    pinned-host hipMemcpyAsync of 1 GiB each way."""
    import numpy as np
    import torch
    from vllm_kv_amd import workloads
    lib = _ceil_lib()
    stream = torch.cuda.current_stream()
    h = stream.cuda_stream
    cus = _cus(dev)
    rows = {}
    # matrix cores: 1, 2 and 4 waves per SIMD (256-thread workgroups, one per CU per wave slot)
    out = torch.empty(cus * 4 * 256, dtype=torch.float32, device=dev)
    iters = 4000
    mf = {}
    for wps in (1, 2, 4):
        blocks = cus * wps
        run = lambda: _ck(lib.vkvc_mfma_loop(out.data_ptr(), blocks, iters, h), "vkvc_mfma_loop")
        _warm(run, 3, min_ms=100.0)
        t = _events_ms(run, 10, stream)
        flops = blocks * 4 * iters * 32 * 16384
        mf[f"{wps}_wave_per_simd"] = round(flops / (t[0] * 1e-3) / 1e12, 1)
    best = max(mf.values())
    rows["mfma"] = {"tflops": best, "by_waves_per_simd": mf, "frac_of_spec": round(best / MFMA_PEAK_TFLOPS, 4),
                    "kernel": f"{iters} x 32 v_mfma_f32_16x16x32_f16 per wave, 8 accumulator chains"}
    # sequential read-only stream
    buf = torch.empty(1 << 32, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    sink = torch.empty(cus * 32 * 256, dtype=torch.int32, device=dev)
    rs = {}
    for mult in (4, 8, 16, 32):
        for nt in (0, 1):
            run = lambda: _ck(lib.vkvc_read_stream(buf.data_ptr(), buf.numel(), sink.data_ptr(), cus * mult, nt, h),
                              "vkvc_read_stream")
            _warm(run, 2, min_ms=50.0)
            t = _events_ms(run, 10, stream)
            rs[f"{cus * mult}wg_{'nt' if nt else 'plain'}"] = round(buf.numel() / (t[0] * 1e-3) / 1e9, 1)
    best = max(rs.values())
    rows["read_stream"] = {"gbs": best, "frac_of_spec": round(best / HBM_PEAK_GBS, 4), "bytes": buf.numel(),
                           "by_shape": rs}
    del buf, sink
    torch.cuda.empty_cache()
    # block gathers of the decode configs' byte sets (whole blocks, every head)
    for name, cfg, elem in (("gather_c2", workloads.config2(), 2), ("gather_c5", workloads.config5(), 1)):
        lay = cfg.layout
        nblk = (lay.context_lens.astype(np.int64) + cfg.block_size - 1) // cfg.block_size
        ids = np.concatenate([lay.block_tables[s, :n] for s, n in enumerate(nblk)]).astype(np.int32)
        bb = cfg.block_size * cfg.num_kv_heads * cfg.head_dim * elem
        pool = torch.empty((2, lay.num_blocks * bb), dtype=torch.uint8, device=dev)
        pool.fill_(3)
        gbs, shape, nbytes = gather_ceiling(dev, pool[0], pool[1], ids, bb, stream, calls=50)
        rows[name] = {"gbs": round(gbs, 1), "frac_of_spec": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes,
                      "blocks": int(ids.shape[0]), "block_bytes": bb, "shape": shape}
        # the decode's own pattern: per (row, 768-token partition, kv head) wave, that
        # head's slice of each token row (codes only for FP8), no math
        P = 768
        S, MB = lay.block_tables.shape
        max_parts = int((int(lay.context_lens.max()) + P - 1) // P)
        hb = cfg.head_dim * elem
        d_bt = torch.from_numpy(lay.block_tables).to(dev)
        d_cl = torch.from_numpy(lay.context_lens).to(dev)
        sink = torch.empty(((S * max_parts * cfg.num_kv_heads + 3) // 4) * 256, dtype=torch.int32, device=dev)
        run = lambda: _ck(lib.vkvc_read_heads(pool[0].data_ptr(), pool[1].data_ptr(), d_bt.data_ptr(), d_cl.data_ptr(),
                                              S, MB, cfg.num_kv_heads, cfg.block_size, cfg.num_kv_heads * hb, hb, P,
                                              max_parts, sink.data_ptr(), h), "vkvc_read_heads")
        _warm(run, 3, min_ms=50.0)
        t = _events_ms(run, 50, stream)
        pbytes = int(lay.context_lens.astype(np.int64).sum()) * cfg.num_kv_heads * hb * 2
        pg = pbytes / (t[0] * 1e-3) / 1e9
        rows[name + "_decode_pattern"] = {"gbs": round(pg, 1), "frac_of_spec": round(pg / HBM_PEAK_GBS, 4),
                                          "bytes": pbytes, "us": round(t[0] * 1e3, 1),
                                          "pattern": f"(row, {P}-token partition, kv head) per wave, "
                                                     f"{hb}-byte head slices, non-temporal"}
        del pool, sink
        torch.cuda.empty_cache()
    # host link: pinned host memory <-> device, hipMemcpyAsync of 1 GiB
    nb = 1 << 30
    host = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
    devb = torch.empty(nb, dtype=torch.uint8, device=dev)
    for direction, (dst, src) in (("h2d", (devb, host)), ("d2h", (host, devb))):
        run = lambda: _ck(lib.vkvc_copy(dst.data_ptr(), src.data_ptr(), nb, h), "vkvc_copy")
        _warm(run, 1, min_ms=50.0)
        t = _events_ms(run, 10, stream)
        gbs = nb / (t[0] * 1e-3) / 1e9
        rows[f"host_{direction}"] = {"gbs": round(gbs, 2), "frac_of_spec": round(gbs / HOST_LINK_GBS, 4),
                                     "us": round(t[0] * 1e3, 1)}
    return {"row": "ceilings", "workload": "measurement kernels of vllm-cpp_amd/bench/ceilings.hip",
            "spec": {"mfma_fp16_tflops": MFMA_PEAK_TFLOPS, "hbm_gbs": HBM_PEAK_GBS, "host_link_gbs": HOST_LINK_GBS},
            **rows}


def suite_c4(dev, steps, warmup):
    """C4: copy_blocks of 4096 (src, dst) pairs over 32 layers x (K, V) of
    [N=8192, bs64, Hkv8, D128] fp16 (random bits), then swap of 2048 blocks to
    pinned host memory and back; bit-exact checks at full size."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config4()
    L, N = cfg.num_layers, cfg.num_blocks
    shape = (L, N, cfg.block_size, cfg.num_kv_heads, cfg.head_dim)
    g = torch.Generator(device=dev).manual_seed(3)
    planes = [torch.empty(shape, dtype=torch.int16, device=dev) for _ in range(2)]
    for pl in planes:
        for l in range(L):
            pl[l].random_(-32768, 32767, generator=g)
    pairs = torch.from_numpy(cfg.copy_pairs).to(dev)
    stream = torch.cuda.current_stream()

    def copy():
        vkv.copy_blocks(planes, pairs, stream=stream)

    for _ in range(max(1, warmup // 2)):
        copy()
    t = _events_ms(copy, max(3, steps // 4), stream)
    src = pairs[:, 0].long()
    dst = pairs[:, 1].long()
    exact = all(torch.equal(pl[l][dst], pl[l][src]) for pl in planes for l in range(L))
    copy_bytes = 2 * int(pairs.shape[0]) * L * 2 * cfg.block_bytes
    copy_gbs = copy_bytes / (t[0] * 1e-3) / 1e9
    # swap: blocks -> pinned host -> other device blocks
    nsw = int(cfg.swap_blocks.shape[0])
    hb = vkv.host_block_bytes(planes)
    host = torch.empty(nsw * hb, dtype=torch.uint8, pin_memory=True)
    out_pairs = torch.from_numpy(np.stack([cfg.swap_blocks, np.arange(nsw, dtype=np.int32)], 1)).to(dev)
    free = np.setdiff1d(np.arange(N, dtype=np.int32), cfg.swap_blocks)[:nsw]
    in_pairs = torch.from_numpy(np.stack([np.arange(nsw, dtype=np.int32), free], 1)).to(dev)
    reps = 3
    torch.cuda.synchronize()
    t_out = _events_ms(lambda: vkv.swap_blocks(planes, host, nsw, out_pairs, 0, stream=stream), reps, stream)
    t_in = _events_ms(lambda: vkv.swap_blocks(planes, host, nsw, in_pairs, 1, stream=stream), reps, stream)
    a = torch.from_numpy(cfg.swap_blocks).long().to(dev)
    b = torch.from_numpy(free).long().to(dev)
    swap_exact = all(torch.equal(pl[l][b], pl[l][a]) for pl in planes for l in range(L))
    swap_bytes = nsw * hb
    beside = _decode_beside_swap(dev, planes, host, nsw, out_pairs, in_pairs, swap_bytes)
    from oracle import oracle
    Ls, Ps = 4, 256
    sub_ids = np.unique(np.concatenate([cfg.copy_pairs[:Ps, 0], cfg.copy_pairs[:Ps, 1]]))
    remap = {int(b): i for i, b in enumerate(sub_ids)}
    sub_pairs = np.array([[remap[int(a_)], remap[int(b_)]] for a_, b_ in cfg.copy_pairs[:Ps]], np.int32)
    sid = torch.from_numpy(sub_ids).long().to(dev)
    host_planes = [np.ascontiguousarray(pl[:Ls][:, sid].cpu().numpy()) for pl in planes]
    sec, reps = _cpu_time(lambda: oracle.copy_blocks(host_planes, sub_pairs))
    cpu_copy_bytes = 2 * Ps * Ls * 2 * cfg.block_bytes
    return {"row": "C4 copy_blocks + swap_blocks", "workload": "32 layers x K,V x [8192, 64, 8, 128] fp16, 4096 copy pairs, 2048 swaps",
            "copy_us_median": round(t[0] * 1e3, 1), "copy_bytes_read_plus_write": copy_bytes,
            "copy_roofline": {"bound": "hbm", "achieved": round(copy_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(copy_gbs / HBM_PEAK_GBS, 4)},
            "copy_bit_exact": bool(exact),
            "swap_bytes_per_direction": swap_bytes,
            "swap_out_gbs": round(swap_bytes / (t_out[0] * 1e-3) / 1e9, 1),
            "swap_in_gbs": round(swap_bytes / (t_in[0] * 1e-3) / 1e9, 1),
            "swap_round_trip_bit_exact": bool(swap_exact),
            "decode_beside_swap": beside,
            "cpu_baseline": {"copy_gbs": round(cpu_copy_bytes / sec / 1e9, 3), "cores": 1, "kind": "port",
                             "sample": f"oracle copy_blocks of {Ps} pairs x {Ls} layers x K,V, {reps} calls"}}


def _decode_beside_swap(dev, planes, host, nsw, out_pairs, in_pairs, swap_bytes, reps=40):
    """C2's decode on the default stream alone, then while a swap of the C4
    blocks runs on a side stream (out, then in): decode us per call each way,
    and each swap's rate while the decodes run (HIP events on each stream)."""
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    cfg = workloads.config2()
    lay = cfg.layout
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    shape = (lay.num_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim)
    kc = _rand_half(shape, g, dev, cfg.sigma)
    vc = _rand_half(shape, g, dev, cfg.sigma)
    q = _rand_half((cfg.num_seqs, cfg.num_heads, cfg.head_dim), g, dev, cfg.sigma)
    out = torch.empty_like(q)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(lay.context_lens).to(dev)
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()

    def decode():
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=main)

    for _ in range(5):
        decode()
    torch.cuda.synchronize()
    res = {"decode_us_alone": round(_events_ms(decode, reps, main)[0] * 1e3, 2)}
    for name, pairs, direction in (("out", out_pairs, 0), ("in", in_pairs, 1)):
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        d0 = torch.cuda.Event(enable_timing=True)
        d1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s0.record(side)
        vkv.swap_blocks(planes, host, nsw, pairs, direction, stream=side)
        s1.record(side)
        d0.record(main)
        for _ in range(reps):
            decode()
        d1.record(main)
        torch.cuda.synchronize()
        res[f"decode_us_beside_swap_{name}"] = round(d0.elapsed_time(d1) / reps * 1e3, 2)
        res[f"decodes_inside_swap_{name}"] = bool(d1.elapsed_time(s1) > 0)
        res[f"swap_{name}_gbs_beside_decode"] = round(swap_bytes / (s0.elapsed_time(s1) * 1e-3) / 1e9, 1)
    res["workload"] = f"C2 decode x {reps} on the default stream; swap of {nsw} C4 blocks on a side stream"
    return res


def suite_shapes(dev, steps, warmup):
    """Decode at shapes outside the benchmark configurations (the reference's
    whole shape domain, src/attention/paged_attention.cu:19-38: any head_dim,
    group size and block size, fp32 tensors), each on C2's 64 sequences
    (ctx U[512,4096], seed 1), and chunked prefill at head_dim 64 (the C1
    model's heads on C3's 8 chunks).  One JSON line with a row per shape."""
    import numpy as np
    import torch
    import vllm_kv_amd as vkv
    from vllm_kv_amd import workloads
    c2 = workloads.config2()
    ctx = c2.layout.context_lens
    S = ctx.shape[0]
    stream = torch.cuda.current_stream()
    rows = []
    # (label, H, Hkv, D, block size, tensor dtype, kernel family)
    shapes = [("reference API: fp32 q / KV / out", 32, 8, 128, 16, torch.float32, "fixed"),
              ("head_dim 80", 32, 8, 80, 16, torch.float16, "generic"),
              ("head_dim 96", 32, 8, 96, 16, torch.float16, "generic"),
              ("head_dim 112", 32, 8, 112, 16, torch.float16, "generic"),
              ("head_dim 80, MHA (Phi-2's heads: H32 / Hkv32)", 32, 32, 80, 16, torch.float16, "generic"),
              ("head_dim 96, MHA (Phi-3-mini's heads: H32 / Hkv32)", 32, 32, 96, 16, torch.float16, "generic"),
              ("group 16 (H32 / Hkv2)", 32, 2, 128, 16, torch.float16, "generic"),
              ("MQA (H32 / Hkv1)", 32, 1, 128, 16, torch.float16, "generic"),
              ("block size 12", 32, 8, 128, 12, torch.float16, "generic"),
              ("block size 24", 32, 8, 128, 24, torch.float16, "generic"),
              ("fixed shape for comparison (C2: H32 / Hkv8 / D128 / bs16)", 32, 8, 128, 16, torch.float16, "fixed")]
    for label, H, Hkv, D, bs, dt, fam in shapes:
        lay = workloads.make_layout(ctx, bs, np.random.default_rng(1))
        g = torch.Generator(device=dev).manual_seed(1)
        kc = (torch.randn((lay.num_blocks, bs, Hkv, D), generator=g, device=dev) * c2.sigma).to(dt)
        vc = (torch.randn((lay.num_blocks, bs, Hkv, D), generator=g, device=dev) * c2.sigma).to(dt)
        q = (torch.randn((S, H, D), generator=g, device=dev) * c2.sigma).to(dt)
        bt = torch.from_numpy(lay.block_tables).to(dev)
        cl = torch.from_numpy(lay.context_lens).to(dev)
        out = torch.empty_like(q)
        scale = 1.0 / float(np.sqrt(D))

        def decode():
            vkv.paged_decode(out, q, kc, vc, bt, cl, scale, stream=stream)

        _warm(decode, warmup, min_ms=100.0)
        t = _events_ms(decode, steps, stream)
        kvb = int(ctx.astype(np.int64).sum()) * Hkv * 2 * D * kc.element_size()
        gbs = kvb / (t[0] * 1e-3) / 1e9
        rows.append({"shape": label, "H": H, "Hkv": Hkv, "D": D, "block_size": bs,
                     "dtype": "f32" if dt == torch.float32 else "f16", "kernels": fam,
                     "us_median": round(t[0] * 1e3, 2), "us_p10_p90": [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)],
                     "kv_bytes": kvb, "gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"[shapes] {label}: {t[0] * 1e3:.1f} us, {gbs:.0f} GB/s")
        del kc, vc, q, out
        torch.cuda.empty_cache()
    # prefill at head_dim 64: Qwen2.5-0.5B heads (H14 / Hkv2 / D64, bs16) on C3's 8 chunks
    c3 = workloads.config3()
    npf = int((c3.q_lens > 1).sum())
    ql = c3.q_lens[:npf]
    cl_np = c3.layout.context_lens[:npf]
    H, Hkv, D, bs = 14, 2, 64, 16
    lay = workloads.make_layout(cl_np, bs, np.random.default_rng(2))
    g = torch.Generator(device=dev).manual_seed(2)
    kc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    vc = _rand_half((lay.num_blocks, bs, Hkv, D), g, dev, 0.3)
    qsl_np = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    q = _rand_half((int(qsl_np[-1]), H, D), g, dev, 0.3)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    cl = torch.from_numpy(cl_np).to(dev)
    qsl = torch.from_numpy(qsl_np).to(dev)
    out = torch.empty_like(q)
    scale = 1.0 / float(np.sqrt(D))
    k8 = torch.empty((lay.num_blocks, bs, Hkv, D), dtype=torch.uint8, device=dev)
    v8 = torch.empty_like(k8)
    ks8 = torch.empty((lay.num_blocks, bs, Hkv), dtype=torch.float32, device=dev)
    vs8 = torch.empty_like(ks8)
    slots = torch.arange(lay.num_blocks * bs, dtype=torch.int32, device=dev)
    vkv.reshape_and_cache(kc.reshape(-1, Hkv, D), vc.reshape(-1, Hkv, D), k8, v8, slots, ks8, vs8)
    keys = sum(int(c3.prior_lens[s]) * int(ql[s]) + int(ql[s]) * (int(ql[s]) + 1) // 2 for s in range(npf))
    flops = 4.0 * D * H * keys
    for label, kk, vv, ksc, vsc in (("prefill head_dim 64, fp16 cache", kc, vc, None, None),
                                    ("prefill head_dim 64, FP8 cache", k8, v8, ks8, vs8)):
        def attn():
            vkv.paged_prefill(out, q, kk, vv, bt, cl, qsl, int(ql.max()), scale, key_scales=ksc,
                              value_scales=vsc, stream=stream, multi_token_only=True)

        _warm(attn, warmup, min_ms=100.0)
        t = _events_ms(attn, steps, stream)
        tf = flops / (t[0] * 1e-3) / 1e12
        rows.append({"shape": label, "H": H, "Hkv": Hkv, "D": D, "block_size": bs, "dtype": "f16",
                     "us_median": round(t[0] * 1e3, 2), "us_p10_p90": [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)],
                     "gflop": round(flops / 1e9, 2), "tflops": round(tf, 1), "frac_of_mfma_peak": round(tf / 2500.0, 4)})
        log(f"[shapes] {label}: {t[0] * 1e3:.1f} us, {tf:.0f} TFLOP/s")
    return {"row": "other shapes", "workload": "decode: C2's 64 sequences (ctx U[512,4096], seed 1) at each shape; "
                                              "prefill: C3's 8 chunks (512 tokens on prior U[0,2048], seed 2) "
                                              "at H14 / Hkv2 / D64",
            "rows": rows}


SUITES = {"ceil": suite_ceilings, "stream": suite_stream, "c1": suite_c1, "append": suite_append, "rope": suite_rope, "step": suite_step,
          "c3": suite_c3,
          "c3p": suite_c3_prefill_only, "c5": suite_c5, "c4": suite_c4, "shapes": suite_shapes}


def run_suite(names, steps, warmup):
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    for name in names:
        log(f"[suite] {name}")
        r = SUITES[name](dev, steps, warmup)
        print(json.dumps(r), flush=True)
        torch.cuda.empty_cache()


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--suite":
        run_suite(sys.argv[2].split(",") if len(sys.argv) > 2 else list(SUITES), 50, 5)
        sys.exit(0)
    main()
