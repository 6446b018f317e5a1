"""Benchmark of the MI355X KV-cache hot path (one JSON line on stdout).

Headline workload (the path's batched serving step):
  32 sequences, lengths drawn U[128, 8192] from seed 3, 32 query / 8 KV heads,
  head_dim 128, fp16 KV in 16-token pages whose physical ids are a seeded
  random permutation of one shared pool.  One step = paged append of one new
  K/V token per sequence at position L_b, then split-K decode attention of one
  query per sequence over L_b + 1 keys, as one kvhp_paged_append_decode call
  (the split covering L_b writes the row and attends it from registers).
  Lengths are held fixed from step to step (each step rewrites the same
  slot), so every timed step does identical work.  The timed steps rotate
  over --pools (default 4) separately allocated copies of the inputs, so no
  step finds the previous step's 504 MB in the 256 MB MALL.

value = algorithmic bytes of the step (decode: K+V of every cached token once,
q read, out write, block-table and length reads; append: new K/V read + write)
divided by the measured step time (host clock over the timed steps).
roofline = that call (split kernel + merge kernel), timed by one HIP event
pair on its stream around the timed region; also against the device's
measured streaming-read ceiling (kvhp_stream_read over 2 GiB, flushed) and
against the paged-read ceiling at the step's own size (kvhp_page_read), and
beside it the same steps on one pool back to back and single flushed steps
(median, min, max).
cpu_baseline = the oracle's restatement of the reference CPU attention
arithmetic (oracle/kvhp_oracle.c) on the same inputs, on the host cores.

Also reported under "extra" (each measured with L2+MALL flushed by a 512 MB
write and a 1 GiB read before every rep unless labelled warm; median, min and
max): config 1 (decode at ctx 512), config 2 (ctx 4K/16K/64K x splits
1/4/16/64, also against the streaming-read ceiling), config 4 (causal prefill
S=512/2048/8192 writing the K/V pages, TFLOP/s vs fp16 MFMA peak, the
attention alone beside it), config 5 (Llama-style 1.1B:
2048-id prefill, then 128 greedy decode steps, tok/s and the HBM bytes of a
step against 8 TB/s; also top-level as config5_decode_tok_s), the same
model serving 8 and 32 sequences per step through the batched runner
(ctx 2048, eager launches, tok/s), and the KV movement kernels alone (paged
gather of the config-3 pool, 2048-token appends).  The line carries the library's build id (source hash) and whether
it matches the sources in the tree.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "serving-engine_amd"))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
METRIC = ("decode-attn HBM GB/s (% of peak) + µs/step; 1.1B decode tok/s at ctx 2K, 1 GPU")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--splits", type=int, default=0, help="decode split count (0 = auto)")
    ap.add_argument("--pools", type=int, default=4,
                    help="separately allocated config-3 input copies the timed steps rotate "
                         "over (504 MB each)")
    ap.add_argument("--no-extra", action="store_true", help="skip configs 1, 2 and 4")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="",
                    help="comma list of extra parts: c1,c2,c4,c5,c5b,kv,layout")
    ap.add_argument("--profile", nargs="?", const="decode", default=None,
                    choices=("decode", "prefill", "c5", "batched", "c2", "kv"),
                    help="short run for rocprofv3: a 256 MiB device copy (counter "
                         "calibration) then the config-3 steps (decode), config-4 "
                         "S=2048 prefill calls (prefill), --steps config-5 decode "
                         "steps without the HIP graph (c5), --steps batched decode "
                         "steps of the config-5 model at B = 1, 8, 32 (batched) or "
                         "--steps flushed config-2 calls (auto splits) per context "
                         "(c2), or the KV movement kernels: paged gather and 2048-token "
                         "appends, flushed and rotating over copies (kv); no CPU "
                         "baseline, no extras")
    return ap.parse_args()


class Flusher:
    """Evicts L2 and MALL (256 MB) between reps: writes 512 MB, then reads
    1 GiB, so the written lines are written back before the timed region
    and the timed kernel does not pay for the flush's own dirty data."""

    def __init__(self, torch):
        self.wbuf = torch.empty(1 << 27, dtype=torch.float32, device="cuda")
        self.buf = torch.ones(1 << 28, dtype=torch.float32, device="cuda")

    def __call__(self):
        self.wbuf.fill_(1.0)
        self.buf.sum()


def time_op(torch, fn, reps, flush=None):
    """Device time (us) of fn over reps: (median, mean, min, max), HIP events
    on the current stream, optional flush before each rep (outside the
    events)."""
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(reps):
        if flush:
            flush()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        fn()
        e.record(stream)
        e.synchronize()
        times.append(s.elapsed_time(e) * 1e3)
    return (float(np.median(times)), float(np.mean(times)), float(np.min(times)),
            float(np.max(times)))


def spread(t, nbytes=None):
    """{median, min, max} of a time_op result in us (and GB/s when nbytes)."""
    d = {"us": round(t[0], 2), "us_min": round(t[2], 2), "us_max": round(t[3], 2)}
    if nbytes:
        d["GB/s"] = round(nbytes / t[0] / 1e3, 1)
    return d


def run_page_read(torch, kvhp, nbytes, page_bytes=4096, reps=25, ordered=False):
    """Ceiling of a paged decode's page reads (kvhp_page_read): a dense pool of
    nbytes read once in a seeded random page order (ordered: address order),
    as the config-3 step reads its pool; flushed before each rep, 5 warm-up
    and `reps` timed reps."""
    n = max(1, nbytes // page_bytes)
    pool = torch.ones((n * page_bytes) // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    order = np.arange(n) if ordered else np.random.default_rng(7).permutation(n)
    ids = torch.from_numpy(order.astype(np.int32)).cuda()
    fl = Flusher(torch)
    for _ in range(5):
        kvhp.page_read(pool, ids, page_bytes, sink)
    t = time_op(torch, lambda: kvhp.page_read(pool, ids, page_bytes, sink), reps, fl)
    rb = n * page_bytes
    del pool, fl
    torch.cuda.empty_cache()
    return {"GBps": round(rb / t[0] / 1e3, 1), "GBps_best": round(rb / t[2] / 1e3, 1),
            "GBps_worst": round(rb / t[3] / 1e3, 1), "bytes": rb, "pages": n,
            "page_bytes": page_bytes, "reps": reps,
            "pct_of_spec": round(rb / t[0] / 1e3 / HBM_PEAK_GBS * 100, 1),
            "kernel": "page_read_kernel (kvhp_page_read), dense pool in %s page order, "
                      "flushed" % ("address" if ordered else "random")}


def run_page_layout(torch, kvhp, reps=20):
    """Is the config-3 step's ceiling the page layout's?  (1) The page-read
    ceiling at the decode's bytes for pages of 2 to 32 KB in random order, and
    4 KB pages in address order; (2) the config-3 step (fused append +
    decode, flushed single calls) with the config's random page tables and
    with each sequence's pages in address order, timed alternately."""
    c = build_config3(torch, kvhp)
    b, hq, hkv, d = c["b"], c["hq"], c["hkv"], c["d"]
    L1 = c["lens"] + 1
    dbytes = decode_bytes(L1, hq, hkv, d)
    del c
    torch.cuda.empty_cache()
    sweep = []
    for pb in (2048, 4096, 8192, 16384, 32768):
        r = run_page_read(torch, kvhp, dbytes, pb, reps)
        sweep.append({"page_bytes": pb, "GBps": r["GBps"], "GBps_best": r["GBps_best"]})
    r = run_page_read(torch, kvhp, dbytes, 4096, reps, ordered=True)
    addr = {"page_bytes": 4096, "GBps": r["GBps"], "GBps_best": r["GBps_best"]}
    max_len = int(L1.max())
    ws_bytes = kvhp.decode_workspace_bytes(b, hq, hkv, d, max_len, 0)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    kvhp.decode_workspace_init(ws)
    fl = Flusher(torch)
    steps = {}
    for name, ordered in (("random", False), ("address", True)):
        ci = build_config3(torch, kvhp, ordered=ordered)
        kv, vv = kvhp.paged_view(ci["pool_k"], ci["bt"]), kvhp.paged_view(ci["pool_v"], ci["bt"])
        nk, nv = ci["new_k"].view(b, hkv, d), ci["new_v"].view(b, hkv, d)

        def fn(ci=ci, kv=kv, vv=vv, nk=nk, nv=nv):
            kvhp.paged_append_decode(ci["q"], nk, nv, kv, vv, ci["pos"], ci["lens1"], ci["out"],
                                     hq, hkv, d, max_len, 0, ws)
        for _ in range(3):
            fn()
        steps[name] = (ci, fn, [])
    for _ in range(3):
        for name in ("random", "address"):
            steps[name][2].append(time_op(torch, steps[name][1], reps // 3 + 1, fl)[0])
    sbytes = dbytes + append_bytes(b, hkv, d)
    res = {}
    for name in ("random", "address"):
        us = float(np.median(steps[name][2]))
        res[name] = {"us": round(us, 2), "GBps": round(sbytes / us / 1e3, 1),
                     "frac": round(sbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                     "us_runs": [round(x, 2) for x in steps[name][2]]}
    del steps, fl, ws
    torch.cuda.empty_cache()
    return {"workload": "config-3 decode bytes (%d B): page-read ceiling by page size (random "
                        "order) and in address order; the config-3 step (kvhp_paged_append_decode, "
                        "flushed single calls, median of 3 alternating runs) with random and "
                        "address-ordered page tables" % dbytes,
            "page_read_random": sweep, "page_read_address_4k": addr, "step": res}


def run_stream_read(torch, kvhp, gib=2, reps=25):
    """The device's achievable streaming-read bandwidth (kvhp_stream_read:
    16-byte non-temporal loads over `gib` GiB, far beyond the 256 MB MALL),
    flushed before each rep, 5 warm-up and `reps` timed reps; the ceiling the
    decode numbers are also reported against (as the reference calibrates
    its decode roofline, docs/GATES.md:21)."""
    buf = torch.ones((gib << 30) // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    fl = Flusher(torch)
    for _ in range(5):
        kvhp.stream_read(buf, sink)
    t = time_op(torch, lambda: kvhp.stream_read(buf, sink), reps, fl)
    nbytes = buf.numel() * 4
    del buf, fl
    torch.cuda.empty_cache()
    return {"GBps": round(nbytes / t[0] / 1e3, 1), "GBps_best": round(nbytes / t[2] / 1e3, 1),
            "GBps_worst": round(nbytes / t[3] / 1e3, 1), "bytes": nbytes, "reps": reps,
            "pct_of_spec": round(nbytes / t[0] / 1e3 / HBM_PEAK_GBS * 100, 1),
            "kernel": "stream_read_kernel (kvhp_stream_read), flushed"}


# ---------------------------------------------------------------- config 3 --
def decode_bytes(lens, hq, hkv, d):
    lens = np.asarray(lens, np.int64)
    kv = int(lens.sum()) * hkv * d * 2 * 2
    qo = 2 * len(lens) * hq * d * 2
    table = int(((lens + 15) // 16).sum()) * 4 + len(lens) * 4
    return kv + qo + table


def append_bytes(b, hkv, d):
    return b * hkv * d * 2 * 2 * 2 + b * 4 * 2


def build_config3(torch, kvhp, seed=3, value_seed=None, ordered=False):
    """Config-3 inputs: lengths and page tables from numpy seed `seed`, K/V
    pool, new rows and q from torch seed `value_seed` (default `seed`).
    ordered: page ids dealt in address order (each sequence's pages
    contiguous in the pool) instead of the config's random permutation."""
    b, hq, hkv, d = 32, 32, 8, 128
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 8193, size=b).astype(np.int32)  # cached tokens
    need = (lens + 1 + 15) // 16
    P = int(need.sum()) + 16
    maxp = int(need.max()) + 1
    perm = rng.permutation(P).astype(np.int32)
    if ordered:
        perm = np.arange(P, dtype=np.int32)
    bt = np.full((b, maxp), -1, np.int32)
    o = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[o:o + n]
        o += int(n)
    dev = torch.device("cuda")
    g = torch.Generator(device="cuda").manual_seed(seed if value_seed is None else value_seed)
    pool_k = torch.randn((hkv, P, 16, d), generator=g, device=dev).half()
    pool_v = torch.randn((hkv, P, 16, d), generator=g, device=dev).half()
    new_k = torch.randn((b, 1, hkv, d), generator=g, device=dev).half()
    new_v = torch.randn((b, 1, hkv, d), generator=g, device=dev).half()
    q = torch.randn((b, hq, d), generator=g, device=dev).half()
    return dict(b=b, hq=hq, hkv=hkv, d=d, lens=lens, bt=torch.from_numpy(bt).to(dev),
                bt_np=bt, P=P, pool_k=pool_k, pool_v=pool_v, new_k=new_k, new_v=new_v, q=q,
                pos=torch.from_numpy(lens).to(dev),
                lens1=torch.from_numpy(lens + 1).to(dev),
                out=torch.empty((b, hq, d), dtype=torch.float16, device=dev))


def host_cpu_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def time_cpu(fn, min_reps, min_seconds):
    """Median seconds of fn over at least min_reps runs (and min_seconds),
    after one warm-up run."""
    fn()
    ts, t_all = [], time.perf_counter()
    while len(ts) < min_reps or time.perf_counter() - t_all < min_seconds:
        t0 = time.perf_counter()
        out = fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts), out


def cpu_baseline_config3(c, torch):
    """Oracle decode (reference attention arithmetic restated in C) on the
    same step's inputs: the full 32-sequence step, median of >= 5 runs after
    a warm-up, on all host threads (up to 16, the box's share) and on one."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    b, hq, hkv, d = c["b"], c["hq"], c["hkv"], c["d"]
    L1 = c["lens"] + 1
    cap = int(L1.max())
    # The oracle's inputs are gathered on the host from the pool and the page
    # tables (not by the GPU gather under test), with each sequence's new
    # row at position L_b taken from the step's own new K/V (not from the
    # GPU's fused append).
    bt = c["bt_np"]
    slot = np.arange(cap) % 16
    page = np.arange(cap) // 16
    kf = np.zeros((b, hkv, cap, d), np.float32)
    vf = np.zeros((b, hkv, cap, d), np.float32)
    new_k = c["new_k"].float().cpu().numpy().reshape(b, hkv, d)
    new_v = c["new_v"].float().cpu().numpy().reshape(b, hkv, d)
    for name, dst, new in (("pool_k", kf, new_k), ("pool_v", vf, new_v)):
        pool = c[name].cpu().numpy()   # [hkv][P][16][d] fp16
        for i in range(b):
            n = int(c["lens"][i])
            dst[i, :, :n, :] = pool[:, bt[i, page[:n]], slot[:n], :]
            dst[i, :, n, :] = new[i]
        del pool
    qf = c["q"].float().cpu().numpy()
    threads = min(16, os.cpu_count() or 1)
    nbytes = decode_bytes(L1, hq, hkv, d)
    med, reps, ref = time_cpu(lambda: oracle.decode_attention(qf, kf, vf, L1, hq, hkv, d, threads),
                              5, 2.0)
    med1, reps1, _ = time_cpu(lambda: oracle.decode_attention(qf, kf, vf, L1, hq, hkv, d, 1), 5, 0.0)
    gpu_out = c["out"].float().cpu().numpy()
    err = float(np.abs(gpu_out - ref).max())
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"full config-3 decode step (32 seqs, sum L={int(L1.sum())}), median of "
                      f"{reps} runs {med * 1e3:.1f} ms; oracle max-abs diff vs GPU output "
                      f"{err:.2e}",
            "us_per_step": round(med * 1e6, 1),
            "one_thread": {"value": round(nbytes / med1 / 1e9, 3), "unit": "GB/s",
                           "us_per_step": round(med1 * 1e6, 1), "runs": reps1},
            **host_cpu_info()}


def cpu_baseline_config5(torch, kvhp, prompt_len=16, steps=6):
    """The decoder oracle (reference CPU forward restated, with a K/V cache)
    on the config-5 model's weights read back from the GPU: a seeded
    prompt_len-id prefill, one untimed warm-up decode step, then `steps`
    timed greedy decode steps (median), all host threads (up to 16).
    Bounded sample: the decode step's cost is dominated by the 2.07 GB of
    weights, not by the short context."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from llama_oracle import LlamaOracle
    cfg = kvhp.llama_1b_config()
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=prompt_len + steps + 1)
    f32 = lambda t: t.astype(np.float32)
    v, hdim, f = cfg.vocab_size, cfg.hidden_size, cfg.ffn_size
    nqkv = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * cfg.head_dim
    w = {"embed": f32(model.tensor(-1, kvhp.LLAMA_EMBED)).reshape(v, hdim),
         "lm_head": f32(model.tensor(-1, kvhp.LLAMA_LM_HEAD)).reshape(v, hdim),
         "final_norm": f32(model.tensor(-1, kvhp.LLAMA_FINAL_NORM)), "layers": []}
    for li in range(cfg.num_layers):
        w["layers"].append({
            "attn_norm": f32(model.tensor(li, kvhp.LLAMA_ATTN_NORM)),
            "ffn_norm": f32(model.tensor(li, kvhp.LLAMA_FFN_NORM)),
            "w_qkv": f32(model.tensor(li, kvhp.LLAMA_W_QKV)).reshape(nqkv, hdim),
            "w_o": f32(model.tensor(li, kvhp.LLAMA_W_O)).reshape(hdim, hdim),
            "w_gate_up": f32(model.tensor(li, kvhp.LLAMA_W_GATE_UP)).reshape(2 * f, hdim),
            "w_down": f32(model.tensor(li, kvhp.LLAMA_W_DOWN)).reshape(hdim, f)})
    model.close()
    threads = min(16, os.cpu_count() or 1)
    ref = LlamaOracle(cfg, w, nthreads=threads)
    prompt = np.random.default_rng(5).integers(0, v, prompt_len).astype(np.int32)
    t0 = time.perf_counter()
    logits = ref.forward(prompt)
    t_prefill = time.perf_counter() - t0
    logits = ref.forward([int(np.argmax(logits))])     # warm-up step, untimed
    per_tok = []
    for _ in range(steps):
        t0 = time.perf_counter()
        logits = ref.forward([int(np.argmax(logits))])
        per_tok.append(time.perf_counter() - t0)
    s_tok = float(np.median(per_tok))
    return {"value": round(1.0 / s_tok, 3), "unit": "tok/s", "s_per_token": round(s_tok, 3),
            "cores": threads, "kind": "port",
            "sample": f"{prompt_len}-id prefill ({t_prefill:.2f} s, reported separately), one "
                      f"warm-up step, then {steps} greedy decode steps, median "
                      f"(min {min(per_tok):.3f} s, max {max(per_tok):.3f} s)",
            "prefill_s": round(t_prefill, 3)}


def run_config3(torch, kvhp, args):
    """The headline: config-3 steps rotating over args.pools separately
    allocated copies of the inputs (same lengths and page tables, own K/V
    pools, rows and queries), so between two uses of one pool the other
    copies stream (pools - 1) x 504 MB through the caches: no step can reuse
    the previous one's data from the 256 MB MALL (the cache-cold rule of the
    baseline's timing).  Beside it: the same steps back to back on one pool,
    and single steps after an explicit flush."""
    R = max(args.pools, 1)
    insts = [build_config3(torch, kvhp, value_seed=3 + 1000 * i) for i in range(R)]
    c = insts[0]
    b, hq, hkv, d = c["b"], c["hq"], c["hkv"], c["d"]
    L1 = c["lens"] + 1
    max_len = int(L1.max())
    # 0 = the library's automatic split choice (per-sequence chunks balanced
    # over the batch on the device, within decode_auto_splits slots)
    splits = args.splits
    ws_bytes = kvhp.decode_workspace_bytes(b, hq, hkv, d, max_len, splits)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    kvhp.decode_workspace_init(ws)
    for ci in insts:
        ci["kview"] = kvhp.paged_view(ci["pool_k"], ci["bt"])
        ci["vview"] = kvhp.paged_view(ci["pool_v"], ci["bt"])
        ci["nk"] = ci["new_k"].view(b, hkv, d)
        ci["nv"] = ci["new_v"].view(b, hkv, d)
    stream = torch.cuda.current_stream()

    def step_on(ci):
        # one call: append the token at position L_b, attend over L_b + 1 keys
        kvhp.paged_append_decode(ci["q"], ci["nk"], ci["nv"], ci["kview"], ci["vview"], ci["pos"],
                                 ci["lens1"], ci["out"], hq, hkv, d, max_len, splits, ws)

    def step():
        step_on(c)

    def append():
        kvhp.paged_append_kv(c["new_k"], c["new_v"], c["pool_k"], c["pool_v"], c["bt"],
                             c["pos"], b, 1, hkv, d)

    def decode():
        kvhp.decode_attention(c["q"], c["kview"], c["vview"], c["lens1"], c["out"], hq, hkv, d,
                              max_len, splits, ws)

    def timed(n, rotate):
        """n steps back to back (pool i % R, or pool 0), one HIP event pair
        on the call's stream around them (no per-step records, whose markers
        would sit between the steps' kernels) and the host clock."""
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for i in range(n):
            step_on(insts[i % R] if rotate else c)
        ev1.record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, ev0.elapsed_time(ev1) * 1e3

    for i in range(args.warmup):
        step_on(insts[i % R])
    torch.cuda.synchronize()
    n = args.steps
    # The timed steps as one HIP graph, replayed (a serving loop captures its
    # decode step; the eager launches of the same steps are timed beside
    # it).  The graph's outputs must equal an eager step's bit for bit.
    graph, graph_ok = None, False
    try:
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap, capture_error_mode="thread_local"):
            for i in range(n):
                step_on(insts[i % R])
        stream.wait_stream(cap)
        torch.cuda.synchronize()
        for ci in insts:
            ci["out"].zero_()
        graph.replay()
        torch.cuda.synchronize()
        from_graph = [ci["out"].clone() for ci in insts[:min(R, n)]]
        for ci in insts[:min(R, n)]:
            ci["out"].zero_()
            step_on(ci)
        torch.cuda.synchronize()
        graph_ok = all(torch.equal(g_out, ci["out"]) for g_out, ci in zip(from_graph, insts))
    except Exception as exc:  # capture unsupported here: eager launches only
        log(f"config3 graph capture failed: {exc}")
        graph = None
    if graph is not None and not graph_ok:
        log("config3 graph outputs differ from eager steps: timing eager launches")

    def timed_graph():
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, ev0.elapsed_time(ev1) * 1e3

    eager_wall, eager_region_us = timed(n, True)
    if graph is not None and graph_ok:
        graph.replay()   # warm replay
        wall, region_us = timed_graph()
    else:
        wall, region_us = eager_wall, eager_region_us
    # per-step spread, from a second pass with an event pair per step
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    for i in range(n):
        ev[i][0].record(stream)
        step_on(insts[i % R])
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    step_us = [s.elapsed_time(e) * 1e3 for s, e in ev]
    same_wall, same_region_us = timed(n, False)
    step_bytes = decode_bytes(L1, hq, hkv, d) + append_bytes(b, hkv, d)
    dbytes = decode_bytes(L1, hq, hkv, d)
    res = {
        "ms_per_step": wall * 1e3 / n,
        "value": step_bytes / (wall / n) / 1e9,
        "launch": "hip_graph" if (graph is not None and graph_ok) else "eager",
        "eager_us_per_step": eager_wall * 1e6 / n,
        "eager_us_region": eager_region_us / n,
        "step_us_region": region_us / n,
        "step_us_median": float(np.median(step_us)),
        "step_us_min": float(np.min(step_us)),
        "step_us_max": float(np.max(step_us)),
        "same_pool_us_region": same_region_us / n,
        "pools": R,
        "decode_bytes": dbytes,
        "step_bytes": step_bytes,
        "splits": splits if splits else
                  f"auto (balanced on the device; workspace for up to "
                  f"{kvhp.decode_auto_splits(b, hkv, d, max_len)} splits per sequence)",
        "sum_L": int(L1.sum()),
        "c": c,
    }
    # flushed (cold L2/MALL) times: the fused step, and for comparison the
    # same step as two calls (append kernel, then decode) and decode alone
    fl = Flusher(torch)
    res["step_flushed"] = time_op(torch, step, 10, fl)
    res["separate_flushed"] = time_op(torch, lambda: (append(), decode()), 10, fl)
    res["decode_only_flushed"] = time_op(torch, decode, 10, fl)
    del fl, graph
    for ci in insts[1:]:
        ci.clear()
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------- extras ----
def run_kv_movement(torch, kvhp):
    """KV movement kernels on their own (flushed): paged gather of the config-3
    pool into contiguous [B][Hkv][cap][D] K and V (bit-exact copy, zeros past
    each length), and a 2048-token prompt's K/V appended into 16-token pages
    (paged) or a head-major cache (contiguous)."""
    c = build_config3(torch, kvhp)
    b, hkv, d = c["b"], c["hkv"], c["d"]
    L1 = c["lens"] + 1
    cap = int(L1.max())
    ok = torch.empty((b, hkv, cap, d), dtype=torch.float16, device="cuda")
    ov = torch.empty_like(ok)
    fl = Flusher(torch)
    gt = time_op(torch, lambda: kvhp.paged_gather_kv(c["pool_k"], c["pool_v"], c["bt"],
                                                     c["lens1"], cap, ok, ov), 10, fl)
    g = gt[0]
    g_read = int(L1.sum()) * hkv * d * 2 * 2
    g_write = b * hkv * cap * d * 2 * 2
    del ok, ov, c
    torch.cuda.empty_cache()
    hkv2, d2 = 8, 128

    def rotating(fn, R, rounds=3):
        """us per call, calls back to back over R input/output copies: R calls
        captured as one HIP graph (eager launches from Python are host-bound
        at these sizes), replayed `rounds` times under HIP events."""
        for i in range(R):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(g, stream=cs):
            for i in range(R):
                fn(i)
        torch.cuda.current_stream().wait_stream(cs)
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(rounds):
            g.replay()
        e1.record()
        e1.synchronize()
        del g
        return e0.elapsed_time(e1) * 1e3 / (rounds * R)

    def append_case(S, flushed):
        """Appends of S tokens x 8 heads x D=128 (K and V), paged (identity
        table from position 0) and contiguous, over R copies totalling more
        than the 256 MB MALL; beside them torch's device copy of the same
        bytes (src -> dst, K and V): the ceiling of a plain copy that size."""
        nb = 2 * S * hkv2 * d2 * 2 * 2
        R = max(3, -(-640_000_000 // nb))
        P = S // 16 + 4
        bt = torch.arange(P, dtype=torch.int32, device="cuda").view(1, P)
        zero = torch.zeros(1, dtype=torch.int32, device="cuda")
        srcs = [(torch.randn((1, S, hkv2, d2), device="cuda").half(),
                 torch.randn((1, S, hkv2, d2), device="cuda").half()) for _ in range(R)]
        pools = [(torch.zeros((hkv2, P, 16, d2), dtype=torch.float16, device="cuda"),
                  torch.zeros((hkv2, P, 16, d2), dtype=torch.float16, device="cuda"))
                 for _ in range(R)]
        caches = [(torch.zeros((hkv2, S, d2), dtype=torch.float16, device="cuda"),
                   torch.zeros((hkv2, S, d2), dtype=torch.float16, device="cuda"))
                  for _ in range(R)]

        def paged(i):
            kvhp.paged_append_kv(srcs[i][0], srcs[i][1], pools[i][0], pools[i][1], bt, zero, 1,
                                 S, hkv2, d2)

        def contig(i):
            kvhp.append_kv(srcs[i][0], srcs[i][1], caches[i][0], caches[i][1], S, 0, hkv2, S,
                           d2)

        def copy(i):
            caches[i][0].view(-1).copy_(srcs[i][0].view(-1))
            caches[i][1].view(-1).copy_(srcs[i][1].view(-1))

        row = {"tokens": S, "bytes": nb, "copies": R}
        for name, fn in (("paged", paged), ("contig", contig), ("torch_copy", copy)):
            us = rotating(fn, R)
            row[name] = {"us": round(us, 2), "GBps": round(nb / us / 1e3, 1)}
        if flushed:
            for name, fn in (("paged", paged), ("contig", contig)):
                t = time_op(torch, lambda: fn(0), 20, fl)[0]
                row[name]["flushed_us"] = round(t, 2)
                row[name]["flushed_GBps"] = round(nb / t / 1e3, 1)
        del srcs, pools, caches
        torch.cuda.empty_cache()
        return row

    a2048 = append_case(2048, True)
    sweep = [append_case(S, False) for S in (8192, 32768)]
    del fl
    torch.cuda.empty_cache()
    a_bytes = a2048["bytes"]
    return {"workload": "paged gather of the config-3 pool (32 seqs, sum L=%d) into contiguous "
                        "K/V [32][8][%d][128]; append of 2048 tokens x 8 heads x D=128 (and "
                        "8192 / 32768 tokens as a size sweep)" % (int(L1.sum()), cap),
            "gather_us": round(g, 2), "gather_us_min": round(gt[2], 2),
            "gather_us_max": round(gt[3], 2), "gather_bytes": g_read + g_write,
            "gather_GBps": round((g_read + g_write) / g / 1e3, 1),
            "paged_append_2048_us": a2048["paged"]["flushed_us"],
            "contig_append_2048_us": a2048["contig"]["flushed_us"], "append_bytes": a_bytes,
            "paged_append_GBps": a2048["paged"]["flushed_GBps"],
            "contig_append_GBps": a2048["contig"]["flushed_GBps"],
            "append_2048": a2048, "append_sweep": sweep,
            "note": "*_append_2048_us: one call after a cache flush, HIP events around it "
                    "(median of 20; includes the launch); append_2048 / append_sweep: calls "
                    "back to back over separately allocated input/output copies (more than "
                    "the 256 MB MALL in all), replayed from one HIP graph, HIP events around "
                    "3 replays; torch_copy = a plain device copy of the same bytes (the "
                    "ceiling of a copy that size)"}


def run_config1(torch, kvhp):
    """BASELINE config 1 as the reference's two calls (append_kv_cache, then
    decode_gqa), and as one kvhp_append_decode call on the same cache viewed
    strided (the covering split writes the row, then attends it); both timed
    warm (100 eager steps back to back), replayed from a HIP graph and as
    flushed single steps.  The fused step's output equals the two calls'."""
    hq, hkv, d, max_seq = 32, 8, 64, 512
    g = torch.Generator(device="cuda").manual_seed(1)
    kc = torch.randn((hkv, max_seq, d), generator=g, device="cuda").half()
    vc = torch.randn((hkv, max_seq, d), generator=g, device="cuda").half()
    kn = torch.randn((1, hkv, d), generator=g, device="cuda").half()
    vn = torch.randn((1, hkv, d), generator=g, device="cuda").half()
    q = torch.randn((1, hq, d), generator=g, device="cuda").half()
    out = torch.empty((1, hq, d), dtype=torch.float16, device="cuda")
    out_f = torch.empty_like(out)
    kview = kvhp.strided_view(kc, hkv * max_seq * d, max_seq * d, d)
    vview = kvhp.strided_view(vc, hkv * max_seq * d, max_seq * d, d)
    pos = torch.tensor([511], dtype=torch.int32, device="cuda")
    lens = torch.tensor([512], dtype=torch.int32, device="cuda")

    def step():
        kvhp.append_kv(kn, vn, kc, vc, 1, 511, hkv, max_seq, d)
        kvhp.decode_gqa(q, kc, vc, out, 512, hq, hkv, max_seq, d)

    def fused():
        kvhp.append_decode(q, kn, vn, kview, vview, pos, lens, out_f, hq, hkv, d, max_seq)

    stream = torch.cuda.current_stream()
    fl = Flusher(torch)

    def timings(fn, dst):
        for _ in range(10):
            fn()
        # warm: 100 steps back to back under one event pair (an event pair and a
        # host wait per step would leave the GPU idle between 15-us steps, so its
        # clocks would drop and "warm" would read slower than flushed)
        warm = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(100):
                fn()
            e1.record(stream)
            e1.synchronize()
            warm.append(e0.elapsed_time(e1) * 1e3 / 100)
        warm_t = (float(np.median(warm)), float(np.mean(warm)), float(np.min(warm)),
                  float(np.max(warm)))
        # The same 100 steps replayed from one HIP graph: launched eagerly, a
        # ~12 us step is bounded by the host's launch rate, not the GPU.  The
        # graph's output must equal an eager step's bit for bit.
        graph_t = None
        try:
            gr = torch.cuda.CUDAGraph()
            cap = torch.cuda.Stream()
            cap.wait_stream(stream)
            with torch.cuda.graph(gr, stream=cap, capture_error_mode="thread_local"):
                for _ in range(100):
                    fn()
            stream.wait_stream(cap)
            torch.cuda.synchronize()
            dst.zero_()
            gr.replay()
            torch.cuda.synchronize()
            from_graph = dst.clone()
            dst.zero_()
            fn()
            torch.cuda.synchronize()
            if torch.equal(from_graph, dst):
                gt = []
                for _ in range(5):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    gr.replay()
                    e1.record(stream)
                    e1.synchronize()
                    gt.append(e0.elapsed_time(e1) * 1e3 / 100)
                graph_t = (float(np.median(gt)), float(np.mean(gt)), float(np.min(gt)),
                           float(np.max(gt)))
            else:
                log("config1 graph output differs from an eager step: not reported")
            del gr
        except Exception as exc:  # capture unsupported here: eager figures only
            log(f"config1 graph capture failed: {exc}")
        cold = time_op(torch, fn, 20, fl)
        r = {"us_per_step_flushed": round(cold[0], 2), "flushed": spread(cold),
             "us_per_step_warm": round(warm_t[0], 2),
             "warm": {**spread(warm_t), "note": "median of 5 runs of 100 back-to-back steps, "
                                                "eager launches"}}
        if graph_t is not None:
            r["us_per_step_graph"] = round(graph_t[0], 2)
            r["graph"] = {**spread(graph_t), "note": "median of 5 replays of one HIP graph of "
                                                     "100 steps"}
        return r

    res = {"workload": "config1: append 1 token at pos 511 + decode ctx 512, 32/8 heads, D=64 "
                       "(the reference's two calls: append_kv_cache, decode_gqa)",
           **timings(step, out), "bytes": decode_bytes([512], hq, hkv, d) + append_bytes(1, hkv, d)}
    res["fused"] = {"workload": "the same step as one kvhp_append_decode call on strided views",
                    **timings(fused, out_f)}
    torch.cuda.synchronize()
    res["fused"]["output_equals_two_calls"] = bool(torch.equal(out, out_f))
    return res


def run_config2(torch, kvhp, stream_gbps=None, splits=(1, 4, 16, 64, 0), reps=15,
                contexts=(4096, 16384, 65536)):
    hq, hkv, d = 32, 8, 128
    fl = Flusher(torch)
    rows = []
    for L in contexts:
        g = torch.Generator(device="cuda").manual_seed(L)
        kc = torch.randn((1, hkv, L, d), generator=g, device="cuda").half()
        vc = torch.randn((1, hkv, L, d), generator=g, device="cuda").half()
        q = torch.randn((1, hq, d), generator=g, device="cuda").half()
        out = torch.empty((1, hq, d), dtype=torch.float16, device="cuda")
        lens = torch.tensor([L], dtype=torch.int32, device="cuda")
        kv = kvhp.strided_view(kc, hkv * L * d, L * d, d)
        vv = kvhp.strided_view(vc, hkv * L * d, L * d, d)
        nb = decode_bytes([L], hq, hkv, d)
        for s in splits:
            ws_b = kvhp.decode_workspace_bytes(1, hq, hkv, d, L, s)
            ws = torch.empty(max(ws_b, 256), dtype=torch.uint8, device="cuda")
            kvhp.decode_workspace_init(ws)

            def fn():
                kvhp.decode_attention(q, kv, vv, lens, out, hq, hkv, d, L, s, ws)

            for _ in range(3):
                fn()
            t = time_op(torch, fn, reps, fl)
            row = {"ctx": L, "splits": s if s else f"auto({kvhp.decode_auto_splits(1, hkv, d, L)})",
                   **spread(t, nb), "pct_hbm": round(nb / t[0] / 1e3 / HBM_PEAK_GBS * 100, 1)}
            if stream_gbps:
                row["pct_stream"] = round(nb / t[0] / 1e3 / stream_gbps * 100, 1)
            rows.append(row)
        del kc, vc
    return {"workload": "config2: B=1, 32/8 heads, D=128, contiguous fp16 KV, flushed", "rows": rows}


def run_config4(torch, kvhp, sizes=(512, 2048, 4096, 8192), reps=10, attention_only=True):
    """causal prefill that writes K/V into 16-token pages as
    it runs (kvhp_flash_prefill_paged, a seeded random page permutation); the
    same prefill without the page writes is reported beside it."""
    hq, hkv, d = 32, 8, 128
    rows = []
    fl = Flusher(torch)
    stream = torch.cuda.current_stream()

    def back_to_back(fn, seconds=0.1):
        # MFMA-bound: timed back to back (the inputs come straight from the
        # projection GEMMs in a serving step, cache-warm).  The chip's clocks
        # ramp up over tens of ms of sustained work (from idle an S=2048 call
        # takes 52-57 us and ~46.5-48 us after ~40 ms), and an idle gap drops
        # them again: so ~`seconds` of the same calls are enqueued first and
        # the 5 timed runs of `reps` calls (one event pair each) right behind
        # them, with no host synchronisation in between.  Returns the
        # (median, mean, min, max) per-call time of the runs and the mean of
        # 5 calls under one event pair made first (the cold start), in us.
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        fn()   # first launch of the section (lazy set-up outside the cold figure)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(5):
            fn()
        e1.record(stream)
        e1.synchronize()
        cold = e0.elapsed_time(e1) * 1e3 / 5
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(5)]
        for _ in range(max(1, int(seconds * 1e6 / max(cold, 1.0)))):
            fn()
        for e0, e1 in evs:
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
        torch.cuda.synchronize()
        warm = [e0.elapsed_time(e1) * 1e3 / reps for e0, e1 in evs]
        return (float(np.median(warm)), float(np.mean(warm)), float(np.min(warm)),
                float(np.max(warm))), cold

    for s in sizes:
        g = torch.Generator(device="cuda").manual_seed(s)
        q = torch.randn((s, hq, d), generator=g, device="cuda").half()
        k = torch.randn((s, hkv, d), generator=g, device="cuda").half()
        v = torch.randn((s, hkv, d), generator=g, device="cuda").half()
        out = torch.empty_like(q)
        npages = (s + 15) // 16
        pool_k = torch.zeros((hkv, npages, 16, d), dtype=torch.float16, device="cuda")
        pool_v = torch.zeros_like(pool_k)
        perm = np.random.default_rng(s).permutation(npages).astype(np.int32)
        bt = torch.from_numpy(perm[None, :].copy()).cuda()

        def paged():
            kvhp.flash_prefill_paged(q, k, v, out, s, hq, hkv, d, 1, pool_k, pool_v, bt)

        def plain():
            kvhp.flash_prefill(q, k, v, out, s, hq, hkv, d, 1)

        flops = 2.0 * d * hq * s * (s + 1)
        pct = lambda us: round(flops / us / 1e6 / FP16_PEAK_TFLOPS * 100, 2)
        t, cold = back_to_back(paged)
        tfl = time_op(torch, paged, reps, fl)
        row = {"S": s, **spread(t), "TFLOP/s": round(flops / t[0] / 1e6, 1),
               "pct_fp16_peak": pct(t[0]),
               "flushed": {**spread(tfl), "pct_fp16_peak": pct(tfl[0])},
               "cold_start": {"us": round(cold, 2), "pct_fp16_peak": pct(cold)}}
        if attention_only:
            ta, _ = back_to_back(plain)
            tafl = time_op(torch, plain, reps, fl)
            row["attention_only"] = {**spread(ta), "pct_fp16_peak": pct(ta[0]),
                                     "flushed": {**spread(tafl), "pct_fp16_peak": pct(tafl[0])}}
        rows.append(row)
    return {"workload": "config4: causal prefill B=1, 32/8 heads, D=128, fp16 in / fp32 acc, "
                        "K/V written into 16-token pages (seeded random page order) as the "
                        "prefill runs (kvhp_flash_prefill_paged); back-to-back calls (median "
                        "of 5 runs) enqueued right behind ~0.1 s of the same calls (the "
                        "clocks settle under sustained load), flushed single calls beside; "
                        "cold_start = 5 calls back to back right after the section's set-up "
                        "(mean); "
                        "attention_only = the same prefill without the page writes",
            "rows": rows}


def config5_step_bytes(cfg, ctx):
    """HBM bytes of one batch-1 decode step at context ctx: every weight once
    (fused q/k/v, o, gate/up, down per layer; LM head; one embedding row;
    norm vectors), the K/V cache of all layers, the new K/V rows."""
    h, d, hq, hkv, f, v, L = (cfg.hidden_size, cfg.head_dim, cfg.num_q_heads, cfg.num_kv_heads,
                              cfg.ffn_size, cfg.vocab_size, cfg.num_layers)
    per_layer = ((hq + 2 * hkv) * d * h + h * hq * d + 2 * f * h + h * f + 2 * h) * 2
    kv = L * 2 * hkv * d * 2 * ctx
    return L * per_layer + v * h * 2 + h * 2 + h * 2 + kv


def run_config5(torch, kvhp, steps=128, prompt_len=2048):
    """random-init Llama-style 1.1B, seeded 2048-id prompt,
    prefill then `steps` greedy decode steps (HIP graph of the step)."""
    cfg = kvhp.llama_1b_config()
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=prompt_len + steps + 1)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, prompt_len).astype(np.int32)
    model.prefill(prompt[:16])                     # warm the library paths (rocBLAS, kernels)
    model.close()
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=prompt_len + steps + 1)
    t0 = time.perf_counter()
    first, _ = model.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    toks, ms = model.generate(steps, use_graph=True)
    model.close()
    # same work launched kernel by kernel (no graph), for the launch-overhead picture
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=prompt_len + steps + 1)
    model.prefill(prompt)
    toks2, ms_eager = model.generate(steps, use_graph=False)
    model.close()
    assert toks[:steps + 1].tolist() == toks2[:steps + 1].tolist(), "graph and eager tokens differ"
    tok_s = steps / (ms / 1e3)
    mean_ctx = prompt_len + (steps + 1) / 2
    nb = config5_step_bytes(cfg, mean_ctx)
    gbps = nb * tok_s / 1e9
    return {"workload": "config5: Llama-style 1.1B (22 x [H 2048, 32/4 heads of 64, SwiGLU 5632], "
                        "vocab 32000, untied LM head, fp16 N(0,0.02) weights, norms 1), seeded "
                        f"{prompt_len}-id prompt, {steps} greedy steps, batch 1, HIP graph per step",
            "decode_tok_s": round(tok_s, 1), "ms_per_token": round(ms / steps, 4),
            "decode_tok_s_no_graph": round(steps / (ms_eager / 1e3), 1),
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_tok_s": round(prompt_len / prefill_s, 1),
            "bytes_per_token": nb, "achieved_GBps": round(gbps, 1),
            "pct_hbm_peak": round(gbps / HBM_PEAK_GBS * 100, 2),
            "roofline_tok_s_at_8TBps": round(HBM_PEAK_GBS * 1e9 / nb, 1),
            "first_tokens": toks[:8].tolist()}


def run_config5_eager(torch, kvhp, steps=32, prompt_len=2048):
    """Config 5 decode steps launched kernel by kernel (no HIP graph), so a
    kernel trace sees every launch of the step (profiling mode)."""
    cfg = kvhp.llama_1b_config()
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=prompt_len + steps + 1)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, prompt_len).astype(np.int32)
    model.prefill(prompt)
    toks, ms = model.generate(steps, use_graph=False)
    model.close()
    return {"steps": steps, "ms_per_token_no_graph": round(ms / steps, 4),
            "first_tokens": toks[:8].tolist()}


def run_config5_batched(torch, kvhp, batches=(1, 8, 32), steps=20, ctx=2048, rounds=3):
    """The config-5 model serving B sequences at once through the batched
    runner (kvhp_llama_decode_paged: caller-owned page pool, one block-table
    row per sequence): every sequence prefilled with a seeded ctx-id prompt,
    then `steps` decode steps per batch size, launched eagerly and replayed
    from one HIP graph of the same steps (same positions and lengths in
    device memory, same attention plan), the two timed alternately `rounds`
    times; the graph's last logits must equal an eager step's bit for bit."""
    cfg = kvhp.llama_1b_config()
    L, hkv, d, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    bmax = max(batches)
    per = (ctx + steps + 15) // 16
    P = bmax * per
    model = kvhp.LlamaModel(cfg, seed=5, max_ctx=max(ctx, bmax))
    pool = torch.zeros(L * 2 * hkv * P * 16 * d, dtype=torch.float16, device="cuda")
    bt = torch.arange(P, dtype=torch.int32, device="cuda").view(bmax, per)
    rng = np.random.default_rng(5)
    first = [model.prefill_paged(rng.integers(0, V, ctx).astype(np.int32), pool, P, bt[b], per)[0]
             for b in range(bmax)]
    logits = torch.empty(bmax, V, dtype=torch.float32, device="cuda")
    nxt = torch.empty(bmax, dtype=torch.int32, device="cuda")
    # step i writes position ctx + i of every row and attends over ctx + i + 1
    # keys; every run of the steps rewrites the same K/V (same tokens)
    pos_all = (ctx + torch.arange(steps, dtype=torch.int32, device="cuda")).view(steps, 1)
    cap_len = ctx + steps
    model.reserve(bmax, cap_len)
    out = {}
    ev = lambda: torch.cuda.Event(enable_timing=True)
    for B in batches:
        toks = torch.tensor(first[:B], dtype=torch.int32, device="cuda")
        pos_b = pos_all.expand(steps, B).contiguous()
        seq_b = pos_b + 1

        def step(i, lg):
            model.decode_paged(toks, pool, P, bt[:B], per, pos_b[i], seq_b[i], cap_len, lg,
                               nxt[:B])

        def eager():
            for i in range(steps):
                step(i, logits[:B])
        for i in range(3):
            step(i, logits[:B])
        torch.cuda.synchronize()
        res = {}
        g = None
        try:
            g = torch.cuda.CUDAGraph()
            cs = torch.cuda.Stream()
            cs.wait_stream(torch.cuda.current_stream())
            with torch.cuda.graph(g, stream=cs, capture_error_mode="thread_local"):
                eager()
            torch.cuda.current_stream().wait_stream(cs)
            g.replay()
            torch.cuda.synchronize()
            ref = torch.empty_like(logits[:B])
            step(steps - 1, ref)
            torch.cuda.synchronize()
            if not torch.equal(ref, logits[:B]):
                res["graph_error"] = "graph logits differ from an eager step"
                g = None
        except Exception as exc:  # capture unsupported here: eager figures only
            res["graph_error"] = str(exc)[:200]
            g = None
        te, tg = [], []
        for _ in range(rounds):
            for fn, acc in ((eager, te), (g.replay if g is not None else None, tg)):
                if fn is None:
                    continue
                e0, e1 = ev(), ev()
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                acc.append(e0.elapsed_time(e1) / steps)
        ms = float(np.median(te))
        res.update({"ms_per_step": round(ms, 4), "tok_s": round(B * 1e3 / ms, 1),
                    "ms_min": round(min(te), 4), "ms_max": round(max(te), 4)})
        if tg:
            gms = float(np.median(tg))
            res["graph"] = {"ms_per_step": round(gms, 4), "tok_s": round(B * 1e3 / gms, 1),
                            "ms_min": round(min(tg), 4), "ms_max": round(max(tg), 4)}
        del g
        out[f"B{B}"] = res
    model.close()
    return {"workload": f"config-5 model, batched runner, ctx {ctx}; {steps} steps launched "
                        "eagerly and the same steps replayed from one HIP graph (graph), timed "
                        f"alternately {rounds} times (median, min, max per step)", **out}


def traffic_from_profile(dbytes):
    """HBM bytes per decode call from the committed rocprofv3 --pmc summary
    (profiles/decode_config3_traffic.json), if present."""
    path = os.path.join(ROOT, "profiles", "decode_config3_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return {"bytes": t.get("hbm_bytes_per_call"), "fetch_bytes": t.get("fetch_bytes"),
            "write_bytes": t.get("write_bytes"),
            "ratio_to_algorithmic": round(t["hbm_bytes_per_call"] / dbytes, 4)
            if t.get("hbm_bytes_per_call") else None,
            "source": "profiles/decode_config3_traffic.json"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design, not built)"}))
        sys.exit(2)
    import torch
    import kvhp
    kvhp.load()
    assert torch.cuda.is_available(), "bench needs a GPU"
    if args.profile:
        args.no_cpu = args.no_extra = True
        # plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch
        # calibrate the counters (256 MiB read + 256 MiB written)
        src = torch.ones(1 << 26, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        if args.profile == "prefill":
            # S=2048 runs the key-split kernel, S=8192 the ping-pong one
            r4 = run_config4(torch, kvhp, sizes=(2048, 8192), reps=args.steps, attention_only=False)
            print(json.dumps({"profile": "prefill", "config4": r4}))
            return
        if args.profile == "c5":
            r5 = run_config5_eager(torch, kvhp, steps=args.steps)
            print(json.dumps({"profile": "c5", "config5": r5}))
            return
        if args.profile == "c2":
            r2 = run_config2(torch, kvhp, splits=(0,), reps=args.steps)
            print(json.dumps({"profile": "c2", "config2": r2}))
            return
        if args.profile == "batched":
            rb = run_config5_batched(torch, kvhp, batches=(1, 8, 32), steps=args.steps)
            print(json.dumps({"profile": "batched", "config5_batched": rb}))
            return
        if args.profile == "kv":
            print(json.dumps({"profile": "kv", "kv_movement": run_kv_movement(torch, kvhp)}))
            return
    log("stream-read ceiling ...")
    sr = run_stream_read(torch, kvhp)
    log("config3 timed steps ...")
    r = run_config3(torch, kvhp, args)
    c = r.pop("c")
    dbytes = r["decode_bytes"]
    sbytes = r["step_bytes"]
    achieved = sbytes / r["step_us_region"] / 1e3
    fl_step, fl_sep, fl_dec = r["step_flushed"], r["separate_flushed"], r["decode_only_flushed"]
    log("paged-read ceiling ...")
    pr = run_page_read(torch, kvhp, dbytes)
    line = {
        "metric": METRIC,
        "value": round(r["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "us_per_step": round(r["ms_per_step"] * 1e3, 2),
        "pct_of_hbm_peak": round(r["value"] / HBM_PEAK_GBS * 100, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1) fp16, seeded (torch generators 3, 1003, ...; lengths numpy "
                "seed 3)",
        "build_id": kvhp.build_id(),
        "build_id_matches_sources": kvhp.build_id() == kvhp.source_build_id(),
        "config": {
            "workload": "BASELINE config 3: batched paged decode step, B=32, L~U[128,8192] "
                        "(seed 3), 32 q / 8 KV heads, D=128, 16-token pages, random-permutation "
                        "block tables; step = paged append 1 token/seq + split-K decode; steps "
                        f"rotate over {r['pools']} separately allocated input copies (no step "
                        "reuses the previous step's data from the 256 MB MALL); the timed steps "
                        "are replayed as one HIP graph (launch = hip_graph; eager launches "
                        "beside)",
            "sum_L": r["sum_L"], "splits": r["splits"], "decode_bytes": dbytes,
            "step_bytes": r["step_bytes"], "pools": r["pools"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(dbytes),
                     "kernel": "decode_splitk_kernel<128,4,true,1,false> (append fused) + "
                               "decode_merge_kernel<128,4,false>: one kvhp_paged_append_decode call",
                     "avg_launch_us": round(r["step_us_region"], 2),
                     "per_step_event_us": {"median": round(r["step_us_median"], 2),
                                           "min": round(r["step_us_min"], 2),
                                           "max": round(r["step_us_max"], 2)},
                     "stream_read": sr,
                     "frac_of_stream_read": round(achieved / sr["GBps"], 4),
                     "paged_read": pr,
                     "frac_of_paged_read": round(achieved / pr["GBps"], 4),
                     "launch": r["launch"],
                     "eager": {"us_per_step": round(r["eager_us_per_step"], 2),
                               "us_region": round(r["eager_us_region"], 2),
                               "GBps": round(sbytes / r["eager_us_per_step"] / 1e3, 1),
                               "frac": round(sbytes / r["eager_us_region"] / 1e3 / HBM_PEAK_GBS, 4)},
                     "same_pool_back_to_back_us": round(r["same_pool_us_region"], 2),
                     "same_pool_back_to_back_GBps": round(sbytes / r["same_pool_us_region"] / 1e3, 1),
                     "flushed": {**spread(fl_step, sbytes),
                                 "frac": round(sbytes / fl_step[0] / 1e3 / HBM_PEAK_GBS, 4)},
                     "separate_calls_flushed": spread(fl_sep, sbytes),
                     "decode_only_flushed": spread(fl_dec, dbytes),
                     "note": "achieved = algorithmic bytes of the step / (HIP-event time of the "
                             "timed region / steps), one call per step, steps rotating over the "
                             "input copies and replayed from one HIP graph (eager = the same "
                             "steps launched one by one); same_pool = the steps back to back on one copy; "
                             "flushed = single steps after a 512 MB write + 1 GiB read (median, "
                             "min, max of 10); separate = the step as kvhp_paged_append_kv + "
                             "kvhp_decode_attention; stream_read = the device's streaming-read "
                             "ceiling (kvhp_stream_read over 2 GiB, flushed); paged_read = a "
                             "dense pool of the decode's size read once in a random 4 KB page "
                             "order (kvhp_page_read, flushed): the ceiling of the step's page "
                             "reads at its size"},
    }
    if not args.no_cpu:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline_config3(c, torch)
    del c
    torch.cuda.empty_cache()
    extra = {}
    parts = set(args.only.split(",")) if args.only else {"c1", "c2", "c4", "c5", "c5b", "kv",
                                                           "layout"}
    if not args.no_extra:
        if "kv" in parts:
            log("kv movement ...")
            extra["kv_movement"] = run_kv_movement(torch, kvhp)
        if "layout" in parts:
            log("page layout ...")
            extra["page_layout"] = run_page_layout(torch, kvhp)
        if "c1" in parts:
            log("config1 ...")
            extra["config1"] = run_config1(torch, kvhp)
        if "c2" in parts:
            log("config2 ...")
            extra["config2"] = run_config2(torch, kvhp, sr["GBps"])
        if "c4" in parts:
            log("config4 ...")
            extra["config4"] = run_config4(torch, kvhp)
        if "c5" in parts:
            log("config5 ...")
            extra["config5"] = run_config5(torch, kvhp)
            line["config5_decode_tok_s"] = extra["config5"]["decode_tok_s"]
            if not args.no_cpu:
                log("config5 cpu baseline ...")
                extra["config5"]["cpu_baseline"] = cpu_baseline_config5(torch, kvhp)
        if "c5b" in parts:
            log("config5 batched runner ...")
            extra["config5_batched"] = run_config5_batched(torch, kvhp, batches=(8, 32), steps=20)
    line["extra"] = extra
    print(json.dumps(line))


if __name__ == "__main__":
    main()
