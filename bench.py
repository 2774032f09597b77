"""Benchmark of the MI355X paged-attention path (one JSON line on stdout).

Headline (BASELINE.json metric, config 2): batched paged decode attention,
64 sequences with context lengths uniform in [128, 4096], 64 query heads /
8 KV heads, head_dim 80, fp16 K/V pages of 16 tokens scattered through a pool
of 1.25x the tokens, fp32 q/out.  One "step" = one vcpp_paged_decode call over
the whole batch (decode kernel + split-K merge).  Three independent pools are
rotated so the 256 MB Infinity Cache cannot serve a step from the previous one.

value = algorithmic bytes per step / measured step time, in TB/s, with every
input resident in HBM.  Algorithmic bytes = K and V pages of every context
token (2 * Hkv * D * 2 B per token) + q and out (fp32) + block-table entries.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]

Every leg warms up with at least its warmup count and at least 50 ms of GPU
work before its timed steps: a fresh MI355X raises its clocks over the first
~30 ms of load, and timing that ramp would under-report.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vllm-cpp_amd"))

HBM_PEAK_TBS = 8.0          # MI355X HBM3E, TB/s
F16_MFMA_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s

H, HKV, D, BS = 64, 8, 80, 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the baseline sample")
    ap.add_argument("--partition", type=int, default=0,
                    help="split-K partition size (0 = library default)")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 4 (long context) and config 5 (int8 mixed) legs")
    ap.add_argument("--config-steps", type=int, default=20)
    ap.add_argument("--c4-partitions", type=lambda x: [int(v) for v in x.split(",")],
                    default=[256, 0], help="config 4 variants: partition sizes (0 = balanced)")
    ap.add_argument("--only", choices=["decode", "prefill", "config1", "config4", "config5", "qkprep", "fp8",
                                       "kvwrite", "dense", "longprefill"],
                    help="run one leg only and print its JSON (for profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the prefill leg (for profiling its kernel)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a device-to-device copy of 1 GiB five times (the known-size "
                         "kernel that rocprofv3 FETCH_SIZE / WRITE_SIZE readings are scaled by)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# decode workload (config 2)

def decode_workload(torch, seed, pools=3):
    g = torch.Generator(device="cpu").manual_seed(seed)
    num_seqs = 64
    ctx = torch.randint(128, 4097, (num_seqs,), generator=g, dtype=torch.int32)
    total = int(ctx.sum())
    nb = math.ceil(1.25 * total / BS)
    nblk = [(int(c) + BS - 1) // BS for c in ctx]
    max_blocks = max(nblk)
    dev = torch.device("cuda:0")
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    sets = []
    for i in range(pools):
        k = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float32).half()
        v = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float32).half()
        perm = torch.randperm(nb, generator=g)
        tables = torch.full((num_seqs, max_blocks), -1, dtype=torch.int32)
        off = 0
        for s, n in enumerate(nblk):
            tables[s, :n] = perm[off:off + n]
            off += n
        sets.append((k, v, tables.to(dev)))
    q = torch.randn((num_seqs, H, D), generator=gd, device=dev, dtype=torch.float32)
    out = torch.empty_like(q)
    bytes_per_step = (total * 2 * HKV * D * 2          # K and V pages (fp16)
                      + num_seqs * H * D * (4 + 4)     # q in, out
                      + sum(nblk) * 4)                 # block-table entries
    return dict(ctx=ctx, ctx_dev=ctx.to(dev), nb=nb, sets=sets, q=q, out=out,
                max_ctx=int(ctx.max()), bytes=bytes_per_step, total_tokens=total, nblk=nblk)


def run_decode_steps(torch, pyvcpp, w, steps, workspace, partition=0):
    pages = [pyvcpp.kv_pages(pyvcpp.KV_F16, k, v, BS, HKV, D, w["nb"], BS * HKV * D)
             for k, v, _ in w["sets"]]
    for i in range(steps):
        j = i % len(pages)
        pyvcpp.paged_decode(pages[j], w["q"], w["out"], w["sets"][j][2], w["ctx_dev"],
                            w["max_ctx"], H, workspace=workspace, partition_size=partition)


# ---------------------------------------------------------------------------
# prefill workload (config 3)

def prefill_workload(torch, seed):
    """8 chunks x 2048 new tokens appended to 1024-token paged prefixes, 64/8
    heads, head_dim 80, fp16 Q/K/V ~ N(0, 0.5), block_size 16, random tables."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    chunks, new, prefix = 8, 2048, 1024
    total = prefix + new
    nblk = (total + BS - 1) // BS
    nb = chunks * nblk
    dev = torch.device("cuda:0")
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    k = (0.5 * torch.randn((nb, BS, HKV, D), generator=gd, device=dev)).half()
    v = (0.5 * torch.randn((nb, BS, HKV, D), generator=gd, device=dev)).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tables = perm.view(chunks, nblk).to(dev)
    q = (0.5 * torch.randn((chunks * new, H, D), generator=gd, device=dev)).half()
    out = torch.empty((chunks * new, H, D), dtype=torch.float32, device=dev)
    q_start = torch.arange(0, chunks * new + 1, new, dtype=torch.int32, device=dev)
    pre = torch.full((chunks,), prefix, dtype=torch.int32, device=dev)
    pairs = chunks * sum(prefix + i + 1 for i in range(new))
    flops = 4 * D * H * pairs
    return dict(k=k, v=v, tables=tables, q=q, out=out, q_start=q_start, prefix=pre, nb=nb,
                new=new, flops=flops, chunks=chunks, prefix_len=prefix)


def run_prefill_steps(pyvcpp, pw, steps):
    pages = pyvcpp.kv_pages(pyvcpp.KV_F16, pw["k"], pw["v"], BS, HKV, D, pw["nb"], BS * HKV * D)
    for _ in range(steps):
        pyvcpp.paged_prefill(pages, pw["q"], pw["out"], pw["tables"], pw["q_start"], pw["prefix"],
                             pw["new"], H)


def bench_prefill(torch, pyvcpp, args):
    pw = prefill_workload(torch, args.seed + 7)
    settle(torch, lambda: run_prefill_steps(pyvcpp, pw, 1), 3)
    t0 = time.perf_counter()
    run_prefill_steps(pyvcpp, pw, args.prefill_steps)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.prefill_steps
    pyvcpp.profile_enable(True)
    run_prefill_steps(pyvcpp, pw, args.prefill_steps)
    torch.cuda.synchronize()
    ms, n = pyvcpp.profile_read(pyvcpp.KERNEL_PREFILL)
    pyvcpp.profile_enable(False)
    k_s = ms / max(n, 1) / 1e3
    value = pw["flops"] / dt / 1e12
    achieved = pw["flops"] / k_s / 1e12
    return {
        "metric": "prefill attn TFLOP/s",
        "value": round(value, 2), "unit": "TFLOP/s", "steps": args.prefill_steps,
        "ms_per_step": round(dt * 1e3, 4),
        "pct_of_mfma_peak": round(100 * value / F16_MFMA_PEAK_TFS, 2),
        "dtype": "f16 Q/K/V, fp32 accumulate, fp32 out",
        "config": {"workload": "BASELINE config 3: 8 chunks x 2048 new tokens on 1024-token paged "
                               "prefixes, causal, 64 q / 8 kv heads, head_dim 80, fp16 N(0,0.5)",
                   "flops_per_step": pw["flops"],
                   "flop_count": "4*D*H per causal-valid (query, key) pair"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": F16_MFMA_PEAK_TFS,
                     "unit": "TFLOP/s", "frac": round(achieved / F16_MFMA_PEAK_TFS, 4),
                     "traffic": read_traffic("prefill_dma_config3_traffic.txt"),
                     "kernel": "prefill_dma_kernel<80>",
                     "kernel_avg_us": round(k_s * 1e6, 1)},
    }


# ---------------------------------------------------------------------------
# config 4: long-context decode; config 5: int8 mixed decode + prefill step

def settle(torch, fn, warmup=3, seconds=0.05):
    """Untimed warmup: at least `warmup` calls and at least `seconds` of GPU
    work, so the timed steps run at the clocks the GPU holds under load (they
    ramp up over the first ~30 ms of work on a fresh box)."""
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < seconds:
        fn()
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def timed(torch, fn, steps, warmup=3):
    settle(torch, fn, warmup)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def random_tables(torch, g, lens, nb, dev):
    nblk = [(int(c) + BS - 1) // BS for c in lens]
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    t = torch.full((len(lens), max(nblk)), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        t[i, :n] = perm[off:off + n]
        off += n
    return t.to(dev), nblk


def bench_config4(torch, pyvcpp, args):
    """16 sequences x 32768 tokens, fp16 pages scattered over a pool of 1.25x
    the tokens, split-K over 256-token partitions (the config's statement) and
    the balanced split (the default); 3 rotating pools."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(args.seed + 40)
    gd = torch.Generator(device=dev).manual_seed(args.seed + 41)
    ctx = torch.full((16,), 32768, dtype=torch.int32)
    nb = int(1.25 * int(ctx.sum()) / BS)
    sets = []
    for _ in range(3):
        k = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float16)
        v = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float16)
        tables, nblk = random_tables(torch, g, ctx.tolist(), nb, dev)
        sets.append((pyvcpp.kv_pages(pyvcpp.KV_F16, k, v, BS, HKV, D, nb, BS * HKV * D), k, v, tables))
    q = torch.randn((16, H, D), generator=gd, device=dev)
    out = torch.empty_like(q)
    ctx_d = ctx.to(dev)
    nbytes = int(ctx.sum()) * 2 * HKV * D * 2 + 16 * H * D * 8 + sum(nblk) * 4
    res = {}
    for part in args.c4_partitions:
        need = pyvcpp.decode_workspace_size(sets[0][0], 16, H, 32768, part)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        i = [0]

        def step():
            pg, _, _, tb = sets[i[0] % 3]
            i[0] += 1
            pyvcpp.paged_decode(pg, q, out, tb, ctx_d, 32768, H, partition_size=part, workspace=ws)
        dt = timed(torch, step, args.config_steps)
        pyvcpp.profile_enable(True)
        for _ in range(args.config_steps):
            step()
        torch.cuda.synchronize()
        kms, kn = pyvcpp.profile_read(pyvcpp.KERNEL_DECODE)
        mms, mn = pyvcpp.profile_read(pyvcpp.KERNEL_MERGE)
        pyvcpp.profile_enable(False)
        ks = kms / max(kn, 1) / 1e3
        res["partition_%d" % part if part else "balanced"] = {
            "ms_per_step": round(dt * 1e3, 4), "TB/s": round(nbytes / dt / 1e12, 4),
            "pct_of_hbm_peak": round(100 * nbytes / dt / 1e12 / HBM_PEAK_TBS, 2),
            "decode_kernel_us": round(ks * 1e6, 1), "merge_kernel_us": round(mms / max(mn, 1) * 1e3, 1),
            "kernel_TB/s": round(nbytes / ks / 1e12, 4)}
    return {"metric": "long-context decode HBM TB/s", "unit": "TB/s",
            "config": {"workload": "BASELINE config 4: 16 seqs x 32768 ctx, 64 q / 8 kv heads, "
                                   "head_dim 80, fp16 pages scattered over a 1.25x pool",
                       "bytes_per_step": nbytes},
            "value": res["balanced"]["TB/s"] if "balanced" in res else None, "variants": res,
            "steps": args.config_steps}


def bench_config5(torch, pyvcpp, args):
    """128 decode sequences (ctx U[1024, 8192]) + 4 prefill chunks of 512 new
    tokens on 1024-token prefixes in one step, int8 pages with fp16 scales
    (quantised on the device by vcpp_write_kv from N(0,1) values)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(args.seed + 50)
    gd = torch.Generator(device=dev).manual_seed(args.seed + 51)
    dctx = torch.randint(1024, 8193, (128,), generator=g, dtype=torch.int32)
    plen = [1024 + 512] * 4
    lens = dctx.tolist() + plen
    nb = math.ceil(1.25 * sum(lens) / BS)
    k8 = torch.empty((nb, BS, HKV, D), dtype=torch.int8, device=dev)
    v8 = torch.empty_like(k8)
    ks = torch.zeros((nb, HKV, BS), dtype=torch.int16, device=dev)
    vs = torch.zeros_like(ks)
    pages = pyvcpp.kv_pages(pyvcpp.KV_I8, k8, v8, BS, HKV, D, nb, BS * HKV * D, ks, vs, HKV * BS)
    chunk = 1 << 16  # fill every slot from fp32 N(0,1) through the device quantiser
    for s0 in range(0, nb * BS, chunk):
        n = min(chunk, nb * BS - s0)
        kf = torch.randn((n, HKV, D), generator=gd, device=dev)
        vf = torch.randn((n, HKV, D), generator=gd, device=dev)
        slots = torch.arange(s0, s0 + n, dtype=torch.int64, device=dev)
        pyvcpp.write_kv(pages, kf, vf, slots)
    tables, nblk = random_tables(torch, g, lens, nb, dev)
    dtab, ptab = tables[:128].contiguous(), tables[128:].contiguous()
    qd = torch.randn((128, H, D), generator=gd, device=dev)
    od = torch.empty_like(qd)
    qp = torch.randn((4 * 512, H, D), generator=gd, device=dev).half()
    op = torch.empty((4 * 512, H, D), dtype=torch.float32, device=dev)
    q_start = torch.arange(0, 4 * 512 + 1, 512, dtype=torch.int32, device=dev)
    prefix = torch.full((4,), 1024, dtype=torch.int32, device=dev)
    dctx_d = dctx.to(dev)
    need = pyvcpp.decode_workspace_size(pages, 128, H, 8192, 0)

    need = max(need, pyvcpp.mixed_workspace_size(pages, 128, H, 8192, ptab.shape[1]))
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)

    def two_launches():
        pyvcpp.paged_decode(pages, qd, od, dtab, dctx_d, 8192, H, workspace=ws)
        pyvcpp.paged_prefill(pages, qp.view(torch.int16), op, ptab, q_start, prefix, 512, H)

    def mixed_step():
        pyvcpp.paged_mixed_step(pages, qd, od, dtab, dctx_d, 8192, qp.view(torch.int16), op, ptab,
                                q_start, prefix, 512, H, workspace=ws)

    def fused_one_launch():  # the opt-in single-launch form of the same call
        os.environ["VCPP_MIXED_FUSED"] = "1"
        try:
            mixed_step()
        finally:
            del os.environ["VCPP_MIXED_FUSED"]

    dbytes = (int(dctx.sum()) * (2 * HKV * D + 2 * HKV * 2) + 128 * H * D * 8
              + sum(nblk[:128]) * 4)
    pairs = 4 * sum(1024 + i + 1 for i in range(512))
    flops = 4 * D * H * pairs
    t_star = max(dbytes / (HBM_PEAK_TBS * 1e12), flops / (F16_MFMA_PEAK_TFS * 1e12))
    variants = {}
    for name, step in (("two_launches", two_launches), ("mixed_step", mixed_step),
                       ("fused_one_launch", fused_one_launch)):
        dt = timed(torch, step, args.config_steps)
        pyvcpp.profile_enable(True)
        for _ in range(args.config_steps):
            step()
        torch.cuda.synchronize()
        times = {k: pyvcpp.profile_read(kid) for k, kid in
                 (("decode", pyvcpp.KERNEL_DECODE), ("merge", pyvcpp.KERNEL_MERGE),
                  ("prefill", pyvcpp.KERNEL_PREFILL), ("mixed", pyvcpp.KERNEL_MIXED))}
        pyvcpp.profile_enable(False)
        us = {k: round(v[0] / max(v[1], 1) * 1e3, 1) for k, v in times.items() if v[1] > 0}
        variants[name] = {"ms_per_step": round(dt * 1e3, 4), "fraction_of_t_star": round(t_star / dt, 4),
                          "kernel_us": us}
        if name == "two_launches":
            variants[name]["decode_TB/s_in_kernel"] = round(dbytes / (us["decode"] * 1e-6) / 1e12, 3)
            variants[name]["prefill_TFLOP/s_in_kernel"] = round(flops / (us["prefill"] * 1e-6) / 1e12, 1)
    dt = variants["mixed_step"]["ms_per_step"] * 1e-3
    return {"metric": "int8 mixed step (vcpp_paged_mixed_step): fraction of T* = max(bytes/8 TB/s, flops/2.5 PF)",
            "value": round(t_star / dt, 4), "unit": "fraction",
            "ms_per_step": round(dt * 1e3, 4), "t_star_ms": round(t_star * 1e3, 4),
            "variants": variants, "steps": args.config_steps,
            "config": {"workload": "BASELINE config 5: 128 decode seqs ctx U[1024,8192] + 4 prefill "
                                   "chunks x 512 on 1024-token prefixes, int8 KV + fp16 scales, GQA 8:1, "
                                   "head_dim 80", "decode_bytes": dbytes, "prefill_flops": flops}}


def bench_long_prefill(torch, pyvcpp, args):
    """Chunked prefill of one long request: one chunk of 512 new tokens on a
    paged prefix of 8K / 32K tokens (64 q / 8 kv heads, head_dim 80, fp16
    pages).  The grid of the unsplit kernel is 128 workgroups on 256 CUs;
    vcpp_paged_prefill_split cuts each tile's keys over several workgroups."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(args.seed + 60)
    gd = torch.Generator(device=dev).manual_seed(args.seed + 61)
    res = {}
    for prefix_len in (8192, 32768):
        lens = [prefix_len + 512]
        nb = math.ceil(1.25 * lens[0] / BS)
        k = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float16)
        v = torch.randn((nb, BS, HKV, D), generator=gd, device=dev, dtype=torch.float16)
        pages = pyvcpp.kv_pages(pyvcpp.KV_F16, k, v, BS, HKV, D, nb, BS * HKV * D)
        tables, _ = random_tables(torch, g, lens, nb, dev)
        q = torch.randn((512, H, D), generator=gd, device=dev).half().view(torch.int16)
        out = torch.empty((512, H, D), dtype=torch.float32, device=dev)
        q_start = torch.tensor([0, 512], dtype=torch.int32, device=dev)
        prefix = torch.tensor([prefix_len], dtype=torch.int32, device=dev)
        need = pyvcpp.prefill_workspace_size(pages, 1, 512, prefix_len, H)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        flops = 4 * D * H * sum(prefix_len + i + 1 for i in range(512))
        row = {}
        for name, fn in (("unsplit", lambda: pyvcpp.paged_prefill(pages, q, out, tables, q_start, prefix, 512, H)),
                         ("split", lambda: pyvcpp.paged_prefill_split(pages, q, out, tables, q_start, prefix,
                                                                      512, prefix_len, H, workspace=ws))):
            dt = timed(torch, fn, args.config_steps)
            row[name] = {"us_per_call": round(dt * 1e6, 1), "TFLOP/s": round(flops / dt / 1e12, 1)}
        row["workspace_bytes"] = need
        res["512_on_%d" % prefix_len] = row
    return {"metric": "long-prefix chunked prefill TFLOP/s (split vs unsplit)", "unit": "TFLOP/s",
            "value": res["512_on_32768"]["split"]["TFLOP/s"], "variants": res,
            "steps": args.config_steps,
            "config": {"workload": "1 chunk x 512 new tokens on an 8K / 32K paged prefix, 64 q / 8 kv "
                                   "heads, head_dim 80, fp16 pages"}}


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own paged_attention() (oracle/_ref, built
# from the reference sources), single-threaded, over a bounded sample of the
# same batch (an FP32 pool holding the decoded fp16 values: identical math).

def cpu_baseline(torch, w, target_s):
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    kind = "reference" if O.ref_available() else "port"
    k, v, tables = w["sets"][0]
    tables = tables.cpu().numpy()
    ctx = w["ctx"].numpy().astype(np.int32)
    q = w["q"].cpu().numpy()
    kf = k.float().cpu().numpy()
    vf = v.float().cpu().numpy()
    if kind == "reference":
        pool = O.RefPool(kf, vf, fp16=False)
        cores = 1
        run = lambda: pool.decode(q, tables, ctx, H)
    else:
        pool = O.Pool(O.ORC_F32, kf, vf)
        cores = os.cpu_count() or 1
        run = lambda: O.decode(pool, q, tables, ctx, H, nthreads=cores)
    # whole config-2 batches, repeated until about target_s of CPU time
    reps, dt = 0, 0.0
    while dt < target_s and reps < 1000:
        t0 = time.perf_counter()
        run()
        dt += time.perf_counter() - t0
        reps += 1
    out = {"value": reps * w["bytes"] / dt / 1e12, "unit": "TB/s", "cores": cores, "kind": kind,
           "host_nproc": os.cpu_count(), "host_cores_usable": len(os.sched_getaffinity(0)),
           "sample": "the full config-2 batch (64 seqs, %d context tokens) x %d repetitions, "
                     "paged_attention() per sequence on an FP32 pool holding the decoded fp16 "
                     "values, %.1f s" % (w["total_tokens"], reps, dt)}
    return out


def cpu_port_threaded(torch, w, target_s):
    """The build's own CPU restatement (oracle/oracle.c, orc_decode_batch)
    threaded over (sequence, head) on the host's cores (at most 16, the box's
    CPU share), on the same config-2 batch."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    k, v, tables = w["sets"][0]
    pool = O.Pool(O.ORC_F32, k.float().cpu().numpy(), v.float().cpu().numpy())
    tables = tables.cpu().numpy()
    ctx = w["ctx"].numpy().astype(np.int32)
    q = w["q"].cpu().numpy()
    cores = max(1, min(16, os.cpu_count() or 1))
    reps, dt = 0, 0.0
    while dt < target_s and reps < 1000:
        t0 = time.perf_counter()
        O.decode(pool, q, tables, ctx, H, nthreads=cores)
        dt += time.perf_counter() - t0
        reps += 1
    return {"value": reps * w["bytes"] / dt / 1e12, "unit": "TB/s", "cores": cores, "kind": "port",
            "host_nproc": os.cpu_count(), "host_cores_usable": len(os.sched_getaffinity(0)),
            "sample": "the full config-2 batch x %d repetitions, oracle threaded over (sequence, head), "
                      "%.1f s" % (reps, dt)}


def cpu_prefill_sample(torch, pw, target_s):
    """The reference's prefill on the host (src/paged_engine.cpp:381-384 runs
    one paged_attention-style pass per position; oracle/_ref's ref_prefill
    calls paged_attention() per query row with seq_len = prefix + i + 1), one
    core, on a bounded sample of config 3: rows 0, 16, 32, ... of chunk 0
    (prefix 1024), an FP32 pool holding the chunk's fp16 K/V values."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    if not O.ref_available():
        return None
    tab = pw["tables"][0].long()
    kf = pw["k"][tab].float().cpu().numpy()   # the chunk's blocks, in table order
    vf = pw["v"][tab].float().cpu().numpy()
    pool = O.RefPool(kf, vf, fp16=False)
    rows = np.arange(0, pw["new"], 16)
    q = pw["q"][rows].float().cpu().numpy()
    tables = np.tile(np.arange(kf.shape[0], dtype=np.int32), (len(rows), 1))
    q_start = np.arange(len(rows) + 1, dtype=np.int32)
    prefix = (pw["prefix_len"] + rows).astype(np.int32)
    flops = 4 * D * H * int(sum(int(p) + 1 for p in prefix))
    reps, dt = 0, 0.0
    while dt < target_s and reps < 100:
        t0 = time.perf_counter()
        pool.prefill(q, tables, q_start, prefix, H)
        dt += time.perf_counter() - t0
        reps += 1
    return {"value": reps * flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "reference",
            "host_nproc": os.cpu_count(),
            "sample": "config 3 chunk 0, %d query rows (every 16th of 2048, prefix 1024 + i), "
                      "paged_attention() per row on an FP32 pool holding the fp16 values, "
                      "%d repetitions, %.1f s" % (len(rows), reps, dt)}


def config1_leg(torch, pyvcpp, target_s):
    """BASELINE config 1 (1 sequence, ctx 512, fp32 q and K/V, 64/8 heads,
    head_dim 80, 32 blocks permuted over 64): GPU latency of one
    vcpp_paged_decode call, and the reference on the host with an FP32 pool
    and with its FP16 pool as is (src/kv_cache_manager.cpp:186-211 converts a
    whole block on every key access), one core each."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    pool = O.make_pool(O.ORC_F32, 101, 64, 8, 80)
    q = O.normal(103, (1, 64, 80))
    table = O.permutation(107, 64)[:32].reshape(1, 32).astype(np.int32)
    ctx = np.array([512], np.int32)
    nbytes = 512 * 2 * HKV * D * 4 + 64 * 80 * 8 + 32 * 4
    dev = torch.device("cuda:0")
    k = torch.from_numpy(pool.k).to(dev)
    v = torch.from_numpy(pool.v).to(dev)
    pages = pyvcpp.kv_pages(pyvcpp.KV_F32, k, v, BS, HKV, D, 64, BS * HKV * D)
    qd = torch.from_numpy(q).to(dev)
    out = torch.empty_like(qd)
    td = torch.from_numpy(table).to(dev)
    cd = torch.from_numpy(ctx).to(dev)
    need = pyvcpp.decode_workspace_size(pages, 1, H, 512, 0)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
    run = lambda: pyvcpp.paged_decode(pages, qd, out, td, cd, 512, H, workspace=ws)
    dt = timed(torch, run, 500)
    res = {"workload": "BASELINE config 1: 1 seq, ctx 512, fp32 q / K/V pages, 64 q / 8 kv heads, "
                       "head_dim 80, 32 blocks over 64", "bytes": nbytes,
           "gpu_us_per_call": round(dt * 1e6, 2), "gpu_TB/s": round(nbytes / dt / 1e12, 4)}
    if O.ref_available() and target_s > 0:
        for name, fp16 in (("cpu_ref_fp32_pool", False), ("cpu_ref_fp16_pool_as_is", True)):
            rp = O.RefPool(pool.k, pool.v, fp16=fp16)
            reps, t = 0, 0.0
            while t < target_s and reps < 100000:
                t0 = time.perf_counter()
                rp.decode(q, table, ctx, H)
                t += time.perf_counter() - t0
                reps += 1
            res[name] = {"us_per_call": round(t / reps * 1e6, 1), "TB/s": nbytes * reps / t / 1e12,
                         "cores": 1, "calls": reps}
    return res


def read_traffic(name):
    """HBM bytes per launch recorded in profiles/<name> (rocprofv3 --pmc
    FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def bench_fp8(torch, pyvcpp, args):
    """Config 2's sequences and tables on FP8 E4M3 pages (the reference's
    KV_FP8 format, written on the device by vcpp_write_kv from the same N(0,1)
    values): 1,280 bytes per context token."""
    w = decode_workload(torch, args.seed, pools=3)
    dev = torch.device("cuda:0")
    sets = []
    nrows = w["nb"] * BS
    slots = torch.arange(nrows, dtype=torch.int64, device=dev)
    for k16, v16, tables in w["sets"]:
        k8 = torch.empty((w["nb"], BS, HKV, D), dtype=torch.uint8, device=dev)
        v8 = torch.empty_like(k8)
        pg = pyvcpp.kv_pages(pyvcpp.KV_FP8, k8, v8, BS, HKV, D, w["nb"], BS * HKV * D)
        pyvcpp.write_kv(pg, k16.float().view(nrows, HKV, D), v16.float().view(nrows, HKV, D), slots)
        sets.append((pg, k8, v8, tables))
    torch.cuda.synchronize()
    need = pyvcpp.decode_workspace_size(sets[0][0], 64, H, w["max_ctx"], 0)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
    it = [0]

    def step():
        pg, _, _, tb = sets[it[0] % 3]
        it[0] += 1
        pyvcpp.paged_decode(pg, w["q"], w["out"], tb, w["ctx_dev"], w["max_ctx"], H, workspace=ws)
    steps = max(args.config_steps, 50)
    dt = timed(torch, step, steps)
    pyvcpp.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms, n = pyvcpp.profile_read(pyvcpp.KERNEL_DECODE)
    mms, mn = pyvcpp.profile_read(pyvcpp.KERNEL_MERGE)
    pyvcpp.profile_enable(False)
    k_s = ms / max(n, 1) / 1e3
    nbytes = (w["total_tokens"] * 2 * HKV * D + 64 * H * D * 8 + sum(w["nblk"]) * 4)
    return {
        "metric": "fp8-page decode HBM TB/s", "value": round(nbytes / dt / 1e12, 4), "unit": "TB/s",
        "ms_per_step": round(dt * 1e3, 4), "steps": steps,
        "config": {"workload": "config 2 sequences (64, ctx U[128,4096]) on FP8 E4M3 pages, 64 q / 8 kv "
                               "heads, head_dim 80", "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(nbytes / k_s / 1e9, 1), "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": round(nbytes / k_s / 1e12 / HBM_PEAK_TBS, 4),
                     "kernel": "decode_page_kernel<fp8,80>", "kernel_avg_us": round(k_s * 1e6, 2),
                     "merge_avg_us": round(mms / max(mn, 1) * 1e3, 2)},
    }


def bench_kvwrite(torch, pyvcpp, args):
    """vcpp_write_kv of config 3's 16384 prefill tokens (8 chunks x 2048 on
    1024-token prefixes): K and V fp32 [16384][8][80] into pages, fp16 (the
    reference's truncating encoder), int8 + scale and FP8.  HBM-bound: every
    fp32 value read once, its encoding written once."""
    dev = torch.device("cuda:0")
    T, chunks, new, prefix = 8 * 2048, 8, 2048, 1024
    nblk = (prefix + new) // BS
    nb = chunks * nblk
    g = torch.Generator(device=dev).manual_seed(args.seed + 70)
    k = torch.randn((T, HKV, D), generator=g, device=dev)
    v = torch.randn((T, HKV, D), generator=g, device=dev)
    perm = torch.randperm(nb, device="cpu").to(torch.int64).view(chunks, nblk)
    pos = torch.arange(new, dtype=torch.int64) + prefix
    slots = torch.cat([perm[c, pos // BS] * BS + pos % BS for c in range(chunks)]).to(dev)
    out = {}
    for name, dt, es in (("fp16", pyvcpp.KV_F16, 2), ("int8", pyvcpp.KV_I8, 1), ("fp8", pyvcpp.KV_FP8, 1)):
        tdt = torch.float16 if es == 2 else torch.uint8
        kp = torch.zeros((nb, BS, HKV, D), dtype=tdt, device=dev)
        vp = torch.zeros_like(kp)
        ks = vs = None
        if dt == pyvcpp.KV_I8:
            ks = torch.zeros((nb, HKV, BS), dtype=torch.float16, device=dev)
            vs = torch.zeros_like(ks)
        pg = pyvcpp.kv_pages(dt, kp, vp, BS, HKV, D, nb, BS * HKV * D, ks, vs, HKV * BS)
        nbytes = 2 * T * HKV * D * (4 + es) + T * 8 + (2 * T * HKV * 2 if dt == pyvcpp.KV_I8 else 0)
        steps = max(args.config_steps, 20)
        dt_s = timed(torch, lambda: pyvcpp.write_kv(pg, k, v, slots), steps)
        out[name] = {"us": round(dt_s * 1e6, 2), "TB/s": round(nbytes / dt_s / 1e12, 3), "bytes": nbytes}
    f = out["fp16"]
    return {
        "metric": "KV page write HBM TB/s", "value": f["TB/s"], "unit": "TB/s",
        "config": {"workload": "config 3 chunk tokens: 16384 x 8 kv heads x 80, K and V fp32 -> pages "
                               "(value: fp16, the reference's truncating encoder)"},
        "roofline": {"bound": "hbm", "achieved": round(f["TB/s"] * 1e3, 1), "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": round(f["TB/s"] / HBM_PEAK_TBS, 4), "kernel": "kv_write_vec8_kernel"},
        "variants": out,
    }


def bench_dense(torch, pyvcpp, args):
    """flash_attention_cuda, the reference's contiguous-KV slot
    (cuda/attention.cu:58-124, query row 0 of each (batch, head)): 16 x 64
    (batch, head) pairs over 4096 contiguous fp32 keys, head_dim 80.  Every K
    and V value is read once and the probabilities written once."""
    dev = torch.device("cuda:0")
    B, Hd, kv, ql = 16, H, 4096, 1
    g = torch.Generator(device=dev).manual_seed(args.seed + 90)
    q = torch.randn((B, Hd, ql, D), generator=g, device=dev)
    k = torch.randn((B, Hd, kv, D), generator=g, device=dev)
    v = torch.randn((B, Hd, kv, D), generator=g, device=dev)
    out = torch.empty((B, Hd, D), device=dev)
    w = torch.empty((B * Hd, kv), device=dev)
    L = pyvcpp.lib()

    def run():
        L.flash_attention_cuda(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), w.data_ptr(),
                               B, Hd, D, ql, kv, None)
    nbytes = B * Hd * (2 * kv * D * 4 + kv * 4 + 2 * D * 4)
    steps = max(args.config_steps, 20)
    dt = timed(torch, run, steps)
    tbs = nbytes / dt / 1e12
    return {"metric": "flash_attention_cuda HBM TB/s", "value": round(tbs, 3), "unit": "TB/s",
            "ms_per_step": round(dt * 1e3, 4), "steps": steps,
            "config": {"workload": "16 x 64 (batch, head) pairs, 4096 contiguous fp32 keys, head_dim 80, "
                                   "query row 0 per pair (the reference slot's semantics)",
                       "bytes_per_step": nbytes},
            "roofline": {"bound": "hbm", "achieved": round(tbs * 1e3, 1), "peak": HBM_PEAK_TBS * 1e3,
                         "unit": "GB/s", "frac": round(tbs / HBM_PEAK_TBS, 4),
                         "kernel": "dense_attention_dma_kernel"}}


def bench_qkprep(torch, pyvcpp, args):
    """Fused q/k norm + RoPE (vcpp_qk_norm_rope) over config 3's 16384 prefill
    tokens: q [16384][64][80], k [16384][8][80] fp32 at positions 1024..3071,
    per-head RMS norm then interleaved rotation, in place.  HBM-bound: every
    element read once and written once (plus positions and the norm weights)."""
    dev = torch.device("cuda:0")
    T = 8 * 2048
    g = torch.Generator(device=dev).manual_seed(args.seed + 60)
    q = torch.randn((T, H, D), generator=g, device=dev)
    k = torch.randn((T, HKV, D), generator=g, device=dev)
    pos = (torch.arange(T, dtype=torch.int32, device=dev) % 2048) + 1024
    i = torch.arange(D // 2, dtype=torch.float32, device=dev)
    inv_freq = 1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / D)
    qw = torch.ones(D, device=dev) + 0.1 * torch.randn(D, generator=g, device=dev)
    kw = torch.ones(D, device=dev) + 0.1 * torch.randn(D, generator=g, device=dev)
    nbytes = 2 * (q.numel() + k.numel()) * 4 + T * 4 + 2 * D * 4 + (D // 2) * 4

    def step():
        pyvcpp.qk_norm_rope(q, k, pos, inv_freq, qw, kw, 1e-6, pyvcpp.ROPE_INTERLEAVED)
    steps = max(args.config_steps, 10)
    dt = timed(torch, step, steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    k_s = e0.elapsed_time(e1) / steps / 1e3
    return {
        "metric": "q/k norm + RoPE HBM TB/s", "value": round(nbytes / dt / 1e12, 3), "unit": "TB/s",
        "ms_per_step": round(dt * 1e3, 4), "steps": steps,
        "config": {"workload": "config 3 tokens: 16384 x (64 q + 8 k heads) x 80 fp32, q_norm/k_norm "
                               "then interleaved RoPE at positions 1024..3071, in place",
                   "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(nbytes / k_s / 1e9, 1), "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": round(nbytes / k_s / 1e12 / HBM_PEAK_TBS, 4),
                     "kernel": "qk_prep_lds_kernel<80>", "kernel_avg_us": round(k_s * 1e6, 2)},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (the paged-attention path has no "
              "multi-GPU leg here); got --gpus %d" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch
    import pyvcpp
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    pyvcpp.lib()
    if args.copy_calibration:
        x = torch.empty(1 << 29, dtype=torch.float16, device="cuda:0").fill_(1.0)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": x.numel() * 2, "copy_bytes_written": y.numel() * 2,
                          "launches": 5}))
        return
    if args.prefill_only or args.only == "prefill":
        print(json.dumps(bench_prefill(torch, pyvcpp, args)))
        return
    if args.only == "config1":
        print(json.dumps(config1_leg(torch, pyvcpp, 0.0)))
        return
    if args.only == "config4":
        print(json.dumps(bench_config4(torch, pyvcpp, args)))
        return
    if args.only == "config5":
        print(json.dumps(bench_config5(torch, pyvcpp, args)))
        return
    if args.only == "qkprep":
        print(json.dumps(bench_qkprep(torch, pyvcpp, args)))
        return
    if args.only == "fp8":
        print(json.dumps(bench_fp8(torch, pyvcpp, args)))
        return
    if args.only == "kvwrite":
        print(json.dumps(bench_kvwrite(torch, pyvcpp, args)))
        return
    if args.only == "dense":
        print(json.dumps(bench_dense(torch, pyvcpp, args)))
        return
    if args.only == "longprefill":
        print(json.dumps(bench_long_prefill(torch, pyvcpp, args)))
        return

    w = decode_workload(torch, args.seed)
    pages0 = pyvcpp.kv_pages(pyvcpp.KV_F16, w["sets"][0][0], w["sets"][0][1], BS, HKV, D, w["nb"],
                             BS * HKV * D)
    need = pyvcpp.decode_workspace_size(pages0, 64, H, w["max_ctx"], args.partition)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda:0")

    run_decode_steps(torch, pyvcpp, w, args.warmup, ws, args.partition)
    settle(torch, lambda: run_decode_steps(torch, pyvcpp, w, 1, ws, args.partition), 0)
    t0 = time.perf_counter()
    run_decode_steps(torch, pyvcpp, w, args.steps, ws, args.partition)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1e3 / args.steps
    value = w["bytes"] / (dt / args.steps) / 1e12

    # Same steps again with per-kernel HIP events on the launch stream.
    pyvcpp.profile_enable(True)
    run_decode_steps(torch, pyvcpp, w, args.steps, ws, args.partition)
    torch.cuda.synchronize()
    dec_ms, dec_n = pyvcpp.profile_read(pyvcpp.KERNEL_DECODE)
    mrg_ms, mrg_n = pyvcpp.profile_read(pyvcpp.KERNEL_MERGE)
    pyvcpp.profile_enable(False)
    dec_avg_s = dec_ms / max(dec_n, 1) / 1e3
    achieved = w["bytes"] / dec_avg_s / 1e12

    result = {
        "metric": "decode attn HBM TB/s (% of peak) + prefill attn TFLOP/s (% fp16 MFMA)",
        "value": round(value, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "dtype_note": "f16 K/V pages and MFMA operands (q split hi/lo), fp32 accumulate, fp32 q/out",
        "data": "synthetic (seeded N(0,1) q/K/V, random block tables)",
        "config": {"workload": "BASELINE config 2: batched paged decode, 64 seqs, ctx U[128,4096], "
                               "64 q / 8 kv heads, head_dim 80, fp16 pages of 16 tokens, pool 1.25x",
                   "num_seqs": 64, "context_tokens": w["total_tokens"],
                   "bytes_per_step": w["bytes"], "pool_rotation": len(w["sets"])},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_TBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved * 1e3, 1), "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_TBS, 4),
                     "traffic": read_traffic("decode_page_config2_traffic.txt"),
                     "kernel": "decode_page_kernel<80>",
                     "kernel_avg_us": round(dec_avg_s * 1e6, 2),
                     "merge_avg_us": round(mrg_ms / max(mrg_n, 1) * 1e3, 2)},
        "prefill": None,
    }
    if args.only == "decode":
        args.no_prefill = args.no_configs = args.no_cpu = True
    if not args.no_prefill:
        result["prefill"] = bench_prefill(torch, pyvcpp, args)
    if not args.no_configs:
        result["config4"] = bench_config4(torch, pyvcpp, args)
        result["config5"] = bench_config5(torch, pyvcpp, args)
        result["long_prefill"] = bench_long_prefill(torch, pyvcpp, args)
        result["qk_prep"] = bench_qkprep(torch, pyvcpp, args)
        result["fp8_decode"] = bench_fp8(torch, pyvcpp, args)
        result["kv_write"] = bench_kvwrite(torch, pyvcpp, args)
        result["dense"] = bench_dense(torch, pyvcpp, args)
    if not args.no_configs:
        result["config1"] = config1_leg(torch, pyvcpp, 0.0 if args.no_cpu else 2.0)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, w, args.cpu_seconds)
        result["cpu_port_threaded"] = cpu_port_threaded(torch, w, min(args.cpu_seconds, 5.0))
        if not args.no_prefill:
            result["cpu_prefill"] = cpu_prefill_sample(torch, prefill_workload(torch, args.seed + 7), 5.0)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))


if __name__ == "__main__":
    main()
