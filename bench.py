#!/usr/bin/env python3
"""Benchmark of the OSCAR INT2 rotated KV-cache attention path on one MI355X.

Default workload (BASELINE config 4a, the headline metric): 8 requests, each with
a 24576-token INT2 history and a 4-token MTP chunk (1 + 3 drafts) with causal
masking among the drafts.  The history is written as a server would leave it
after prefill + decode: a standalone KV update of positions [0, L-256) (which
tags no window seat), then a forward write of the last 256 positions with
seq = L, so every request's recent window is held in FP32 (minus the seats
where two requests' window pages hash to the same staging row); Hq=6, Hk=1,
D=256, 128-token pages, random block tables, random-sign Hadamard rotations.  One step = one FULL layer's
forward for the batch: write the 32 new tokens (rotate, INT2 store, window,
rotated q/k/v), split-K attention + LSE merge, inverse rotation to bf16.  The
step cycles over 16 distinct layer caches (1.6 GB, beyond the 256 MB Infinity
Cache) and is replayed from a HIP graph.

Prints one JSON line: whole-step KV-token throughput, the roofline of the
dominant kernel (attn_main: algorithmic bytes / its HIP-event-timed duration)
and a CPU baseline (the NumPy oracle of the same step on this host).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = Path(__file__).resolve().parent / "profiles" / "attn_main_8x24k_mtp_traffic.txt"
LAYERS = 16
CONFIG = dict(requests=8, history=24576, q_len=4, hq=6, hk=1, d=256, block_size=128,
              sink_tokens=64, recent_tokens=256, staging_tokens=8192,
              k_clip=0.0, v_clip=0.0)  # sort-clip ratios of the step's write (--clip: the serve defaults)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def outlier_kv(n, hk, d, gen, dev):
    x = torch.randn(n, hk, d, generator=gen, device=dev)
    ch = torch.randperm(d, generator=gen, device=dev)[:4]
    x[..., ch] *= 8
    return x.bfloat16()


def hadamard_rotation(d, gen, dev):
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < d:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    s = torch.where(torch.rand(d, generator=torch.Generator().manual_seed(7)) < 0.5, -1.0, 1.0)
    return (s.double()[:, None] * h / math.sqrt(d)).float().to(dev).contiguous()


class Setup:
    """Layers of packed caches + staging arenas and one step's static inputs.

    histories: per-request INT2 history lengths; q_len new (or, cache-only, last
    cached) tokens per request.  The history of each request is written as a server
    leaves it: a standalone KV update of all but its last `recent` tokens, then a
    window write of those (so the FP32 recent window is live)."""

    def __init__(self, dev, histories=None, q_len=None, has_new=True, layers=LAYERS, seed=20261201):
        from oscar_amd import ops
        from oscar_amd._lib import STAGE_INVALIDATE, STAGE_WRITE

        c = CONFIG
        histories = histories or [c["history"]] * c["requests"]
        B = len(histories)
        # new tokens (or cache-only queries) per request: one count, or one per request
        ns = [int(x) for x in q_len] if isinstance(q_len, (list, tuple)) else [q_len or c["q_len"]] * B
        n, total = ns[0], sum(ns)
        hq, hk, d, bs = c["hq"], c["hk"], c["d"], c["block_size"]
        self.dev, self.n, self.has_new, self.histories = dev, n, has_new, list(histories)
        gen = torch.Generator(device=dev).manual_seed(seed)
        span = [L + (nr if has_new else 0) for L, nr in zip(histories, ns)]
        pages = [math.ceil(x / bs) for x in span]
        self.nb = sum(pages)
        perm = torch.randperm(self.nb, generator=gen, device=dev).to(torch.int32)
        self.bt = torch.zeros(B, max(pages), dtype=torch.int32, device=dev)
        o = 0
        for r, p in enumerate(pages):
            self.bt[r, :p] = perm[o:o + p]
            o += p
        self.rk = hadamard_rotation(d, gen, dev)
        self.rv = hadamard_rotation(d, gen, dev).flip(0).contiguous()
        self.scale = d ** -0.5
        self.sink_eff = (c["sink_tokens"] // bs) * bs
        rows = max(math.ceil(c["staging_tokens"] / bs),
                   self.sink_eff // bs + math.ceil(c["recent_tokens"] / bs) + 1 + 2)
        recent = c["recent_tokens"]
        body_slots, tail_slots, tail_len = [], [], []
        for r, L in enumerate(histories):
            pos = torch.arange(L, device=dev)
            sl = self.bt[r, pos // bs].long() * bs + pos % bs
            cut = max(L - recent, 0)
            body_slots.append(sl[:cut])
            tail_slots.append(sl[cut:])
            tail_len.append(L - cut)
        body_slots, tail_slots = torch.cat(body_slots), torch.cat(tail_slots)
        qsl_t = torch.tensor([0] + np.cumsum(tail_len).tolist(), dtype=torch.int32, device=dev)
        seq_t = torch.tensor(histories, dtype=torch.int32, device=dev)
        nbody, ntail = body_slots.numel(), tail_slots.numel()
        self.layers = []
        for layer in range(layers):
            kc = torch.zeros(self.nb, bs, hk, d, dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            stage = (torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                     torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                     torch.full((rows, bs), -1, dtype=torch.int64, device=dev))
            for lo in range(0, nbody, 1 << 20):  # standalone KV update of the prefixes
                hi = min(lo + (1 << 20), nbody)
                ops.store(outlier_kv(hi - lo, hk, d, gen, dev), outlier_kv(hi - lo, hk, d, gen, dev), kc, vc,
                          body_slots[lo:hi], head_dim=d, rk=self.rk, rv=self.rv, stage=stage,
                          stage_mode=STAGE_INVALIDATE)
            ops.store(outlier_kv(ntail, hk, d, gen, dev), outlier_kv(ntail, hk, d, gen, dev), kc, vc,
                      tail_slots, head_dim=d, rk=self.rk, rv=self.rv, stage=stage,
                      stage_mode=STAGE_WRITE, qsl_dev=qsl_t, seqs_dev=seq_t, num_reqs=B,
                      recent_tokens=recent, sink_tokens_eff=self.sink_eff)
            self.layers.append((kc, vc, stage))
        torch.cuda.synchronize()
        # step inputs: n new tokens per request at positions L..L+n-1 (or, cache-only,
        # n queries over the cached history)
        self.q = torch.randn(total, hq, d, generator=gen, device=dev).bfloat16()
        self.qsl = [0] + np.cumsum(ns).tolist()
        self.q_rot = torch.empty_like(self.q)
        if has_new:
            self.k_new = outlier_kv(total, hk, d, gen, dev)
            self.v_new = outlier_kv(total, hk, d, gen, dev)
            sl = []
            for r, (L, nr) in enumerate(zip(histories, ns)):
                npos = torch.arange(L, L + nr, device=dev)
                sl.append(self.bt[r, npos // bs].long() * bs + npos % bs)
            self.slots = torch.cat(sl).contiguous()
            self.seqs = [L + nr for L, nr in zip(histories, ns)]
            self.k_rot = torch.empty_like(self.k_new)
            self.v_rot = torch.empty_like(self.v_new)
        else:
            self.k_new = self.v_new = self.k_rot = self.v_rot = None
            self.seqs = list(histories)
        self.qsl_dev = torch.tensor(self.qsl, dtype=torch.int32, device=dev)
        self.seq_dev = torch.tensor(self.seqs, dtype=torch.int32, device=dev)
        self.out_rot = torch.zeros(total, hq, d, dtype=torch.float32, device=dev)
        self.lse = torch.zeros(total, hq, dtype=torch.float32, device=dev)
        self.out = torch.empty(total, hq, d, dtype=torch.bfloat16, device=dev)
        self.plan = None
        if len(set(ns)) == 1 and n * (hq // hk) <= 32:  # decode-shaped: the split-K plan of the step
            self.plan = ops.plan_decode(self.qsl, self.seqs, has_new=has_new, num_kv_heads=hk,
                                        group=hq // hk, head_dim=d, device=dev,
                                        window=(self.sink_eff, c["recent_tokens"]))

    def step(self, layer, phases=0):
        from oscar_amd import ops
        from oscar_amd._lib import STAGE_WRITE

        c = CONFIG
        kc, vc, stage = self.layers[layer]
        store = None
        if self.has_new:
            # the write and the decode in one call (oscar_decode_write_v1)
            store = ops.store_args(self.k_new, self.v_new, kc, vc, self.slots, head_dim=c["d"], rk=self.rk,
                                   rv=self.rv, k_clip=c["k_clip"], v_clip=c["v_clip"], stage=stage, stage_mode=STAGE_WRITE, qsl_dev=self.qsl_dev,
                                   seqs_dev=self.seq_dev, num_reqs=len(self.seqs),
                                   recent_tokens=c["recent_tokens"], sink_tokens_eff=self.sink_eff, query=self.q,
                                   query_rot=self.q_rot, key_rot=self.k_rot, value_rot=self.v_rot)
        else:
            ops.rotate(self.q, self.rk, out=self.q_rot)
        self.attention(layer, store=store)
        ops.rotate(self.out_rot, self.rv, transpose=True, out_dtype=torch.bfloat16, out=self.out)

    def attention(self, layer, phases=0, store=None):
        from oscar_amd import ops

        kc, vc, stage = self.layers[layer]
        ops.attention_decode(self.q_rot, self.k_rot, self.v_rot, kc, vc, self.bt, self.plan,
                             self.scale, stage, head_dim=CONFIG["d"], out_rot=self.out_rot,
                             lse=self.lse, phases=phases, store=store)

    def staged_counts(self):
        """Per-request count of history tokens whose owner tag selects the FP32 window."""
        c = CONFIG
        _, _, (_, _, owner) = self.layers[0]
        own = owner.cpu().numpy()
        bt = self.bt.cpu().numpy().astype(np.int64)
        bs = c["block_size"]
        counts = []
        for r, L in enumerate(self.histories):
            pos = np.arange(L)
            blk = bt[r, pos // bs]
            counts.append(int((own[blk % own.shape[0], pos % bs] == blk).sum()))
        return counts

    def algorithmic_bytes(self, staged):
        """Unique bytes the attention pass must touch (history codes+meta, staged FP32
        window, page-table entries, q, current k/v, owner tags) and the op's outputs."""
        c = CONFIG
        n, hq, hk, d, bs = self.n, c["hq"], c["hk"], c["d"], c["block_size"]
        per_req = [136 * L + 2048 * s + 4 * math.ceil(L / bs) + 2 * n * hq * d
                   + (4 * n * hk * d if self.has_new else 0)
                   for L, s in zip(self.histories, staged)]
        owner = 8 * math.ceil(c["staging_tokens"] / bs) * bs
        b_main = sum(per_req) + owner
        b_out = len(self.histories) * n * hq * (2 * d + 4)
        return b_main, b_main + b_out


def capture(fn_steps, stream=None):
    """A HIP graph of fn_steps() (captured on a side stream, torch's rule for capture)."""
    graph = torch.cuda.CUDAGraph()
    stream = stream or torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            fn_steps()
    torch.cuda.current_stream().wait_stream(stream)
    return graph


def time_graph(setup, steps, warmup):
    """Whole-step time: exactly `steps` layer steps (cycling the layer caches) captured in
    one HIP graph; `warmup` untimed steps (graph replays), then one timed replay of the
    `steps` steps between synchronizations.  Returns (ms per step, steps timed, the
    per-step ms of 5 further replays)."""
    nl = len(setup.layers)
    for i in range(nl):  # eager first use of every layer (lazy state, plans)
        setup.step(i)
    torch.cuda.synchronize()
    graph = capture(lambda: [setup.step(i % nl) for i in range(steps)])
    for _ in range(max(1, math.ceil(warmup / steps))):
        graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    extra = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        extra.append(e0.elapsed_time(e1) / steps)
    return ms, steps, extra


def time_main_kernel(setup, reps=10):
    """Average attn_main duration: a HIP graph of the split-K pass over every layer,
    replayed back to back and bracketed by events on the launch stream (the per-launch
    period includes the short gap between graph nodes)."""
    nl = len(setup.layers)
    for layer in range(nl):
        setup.attention(layer, phases=1)
    torch.cuda.synchronize()
    graph = capture(lambda: [setup.attention(layer, phases=1) for layer in range(nl)])
    graph.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        per.append(e0.elapsed_time(e1) / nl)
    per = np.array(per)
    return float(np.median(per)), float(per.mean())


def event_ms(fn, reps=20, warm=3):
    """Median duration (ms) of fn(r) bracketed by events behind a spin kernel."""
    durs = []
    for r in range(reps + warm):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        e0.record()
        fn(r)
        e1.record()
        e1.synchronize()
        if r >= warm:
            durs.append(e0.elapsed_time(e1))
    return float(np.median(durs))


def config_decode(dev, name, histories, q_len, has_new, layers, steps, warmup):
    """Decode-shaped configs (3, 4b): whole-step KV-token throughput + attn_main roofline."""
    setup = Setup(dev, histories, q_len, has_new, layers)
    staged = setup.staged_counts()
    b_main, _ = setup.algorithmic_bytes(staged)
    ms_step, nsteps, _ = time_graph(setup, steps, warmup)
    med_ms, _ = time_main_kernel(setup)
    achieved = b_main / (med_ms * 1e-3) / 1e9
    kv_tokens = sum(setup.seqs)
    return {"metric": f"INT2-KV attention tokens/s, {name}, one MI355X", "value": kv_tokens / (ms_step * 1e-3),
            "unit": "KV-tokens/s", "n_gpus": 1, "steps": nsteps, "warmup": warmup, "ms_per_step": ms_step,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int2-kv/bf16",
            "data": "synthetic",
            "config": {"workload": name, "requests": len(histories), "history_total": sum(histories),
                       "q_len": q_len, "has_new": has_new, "layers_cycled": layers,
                       "staged_total": sum(staged), "clip": [CONFIG["k_clip"], CONFIG["v_clip"]]},
            "roofline": {"bound": "hbm", "kernel": "attn_main_kernel<256>", "achieved": achieved,
                         "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                         "algorithmic_bytes": b_main, "kernel_us": med_ms * 1e3, "traffic": None}}


def config_store(dev, reps=20, layers=4):
    """Config 2: rotate + INT2 quantize + pack + scatter + FP32 window of 15360 tokens
    (Hk 1, D 256) through a seeded shuffled slot_mapping, 5 % -1 and 2 % rewrites."""
    from oscar_amd import ops
    from oscar_amd._lib import STAGE_WRITE

    c = CONFIG
    N, hk, d, bs = 15360, 1, 256, c["block_size"]
    gen = torch.Generator(device=dev).manual_seed(20261202)
    g = np.random.default_rng(20261202)
    nb = 2 * math.ceil(N / bs)
    slots = g.permutation(nb * bs)[:N].astype(np.int64)
    slots[g.random(N) < 0.05] = -1
    for i in np.nonzero(g.random(N) < 0.02)[0]:
        if i > 0:
            slots[i] = slots[g.integers(0, i)]
    k, v = outlier_kv(N, hk, d, gen, dev), outlier_kv(N, hk, d, gen, dev)
    rk, rv = hadamard_rotation(d, gen, dev), hadamard_rotation(d, gen, dev).flip(0).contiguous()
    rows = max(math.ceil(c["staging_tokens"] / bs), math.ceil(c["recent_tokens"] / bs) + 3)
    sink_eff = (c["sink_tokens"] // bs) * bs
    sl = torch.from_numpy(slots).to(dev)
    qsl = torch.tensor([0, N], dtype=torch.int32, device=dev)
    seqs = torch.tensor([N], dtype=torch.int32, device=dev)
    caches = []
    for _ in range(layers):
        kc = torch.zeros(nb, bs, hk, d, dtype=torch.int8, device=dev)
        caches.append((kc, torch.zeros_like(kc),
                       (torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                        torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                        torch.full((rows, bs), -1, dtype=torch.int64, device=dev))))

    def call(r):
        kc, vc, stage = caches[r % layers]
        ops.store(k, v, kc, vc, sl, head_dim=d, rk=rk, rv=rv, k_clip=c["k_clip"], v_clip=c["v_clip"],
                  stage=stage, stage_mode=STAGE_WRITE, qsl_dev=qsl, seqs_dev=seqs, num_reqs=1,
                  recent_tokens=c["recent_tokens"], sink_tokens_eff=sink_eff)

    ms = event_ms(call, reps)
    valid = slots >= 0
    uniq = len(np.unique(slots[valid]))
    # kept seats: the last writer of each seat is in the recent window (positions >= N - 256)
    seat = (slots // bs % rows) * bs + slots % bs
    last = {}
    for t in np.nonzero(valid)[0]:
        last[int(seat[t])] = t
    kept = sum(1 for t in last.values() if t >= N - c["recent_tokens"] or t < sink_eff)
    # algorithmic bytes: K and V in (bf16), R_k and R_v, slot_mapping, the winners' slot
    # bytes (meta + codes) and claims, the kept FP32 window rows
    b_alg = 2 * N * 512 + 2 * d * d * 4 + 8 * N + 136 * uniq + 8 * uniq + 2048 * kept
    # MFMA work of the rotation: one bf16 x plane against R's two fp16 planes
    flops = 2 * N * 2 * d * d * 2
    t = ms * 1e-3
    return {"metric": "KV store tokens/s (rotate + INT2 pack + scatter + window), config 2, one MI355X",
            "value": N / t, "unit": "tokens/s", "n_gpus": 1, "steps": reps, "warmup": 3, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16 in, f16-MFMA rotation certified against the exact fp32 rotation, int2 out",
            "data": "synthetic",
            "config": {"workload": "config 2: 15360 tokens, 5% -1 slots, 2% rewrites, window write",
                       "clip": [c["k_clip"], c["v_clip"]],
                       "unique_slots": uniq, "kept_window_seats": kept},
            "roofline": {"bound": "hbm", "kernel": "store_prep_kernel + store_fused_kernel + store_exact_kernel",
                         "achieved": b_alg / t / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": b_alg / t / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": b_alg,
                         "mfma_tflops": flops / t / 1e12, "traffic": None}}


def config_prefill(dev, reps=5, layers=2):
    """Config 5: long continuation (15360 INT2 history + 9256-token causal chunk, MFMA
    path) and the history-free 2048-token prefill."""
    from oscar_amd import ops

    c = CONFIG
    hist, nq, hq, hk, d = 15360, 9256, c["hq"], c["hk"], c["d"]
    setup = Setup(dev, [hist], q_len=1, has_new=True, layers=layers, seed=20261205)
    gen = torch.Generator(device=dev).manual_seed(20261206)
    q = torch.randn(nq, hq, d, generator=gen, device=dev).bfloat16()
    k, v = outlier_kv(nq, hk, d, gen, dev), outlier_kv(nq, hk, d, gen, dev)
    out = torch.empty(nq, hq, d, dtype=torch.float32, device=dev)
    lse = torch.empty(nq, hq, dtype=torch.float32, device=dev)
    bs = c["block_size"]
    row = torch.zeros(math.ceil((hist + nq) / bs), dtype=torch.int32, device=dev)
    row[:setup.bt.shape[1]] = setup.bt[0]

    def cont(r):
        kc, vc, stage = setup.layers[r % layers]
        ops.attention_prefill(q, k, v, setup.scale, head_dim=d, history=hist, k_cache=kc, v_cache=vc,
                              block_table_row=row, stage=stage, out=out, lse=lse)

    ms = event_ms(cont, reps, warm=1)
    flops = 4 * d * hq * (nq * hist + nq * (nq + 1) // 2)
    nf = 2048
    qf = torch.randn(nf, hq, d, generator=gen, device=dev).bfloat16()
    kf, vf = outlier_kv(nf, hk, d, gen, dev), outlier_kv(nf, hk, d, gen, dev)
    outf = torch.empty(nf, hq, d, dtype=torch.bfloat16, device=dev)
    ms_f = event_ms(lambda r: ops.attention_prefill(qf, kf, vf, setup.scale, head_dim=d, out=outf), reps, warm=1)
    flops_f = 4 * d * hq * (nf * (nf + 1) // 2)
    t = ms * 1e-3
    return {"metric": "continuation prefill TFLOP/s (15360 INT2 history + 9256 causal), config 5, one MI355X",
            "value": flops / t / 1e12, "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 1,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "config 5: continuation 15360 + 9256; fresh-only 2048",
                       "fresh_2048_ms": ms_f, "fresh_2048_tflops": flops_f / (ms_f * 1e-3) / 1e12},
            "roofline": {"bound": "mfma", "kernel": "prefill_kernel<256>", "achieved": flops / t / 1e12,
                         "peak": 2500.0, "unit": "TFLOP/s", "frac": flops / t / 1e12 / 2500.0,
                         "algorithmic_flops": flops}}


class _Layer:
    layer_name = "model.layers.0.self_attn.attn"


class _Meta:
    pass


def forward_call(setup, layer_idx=0):
    """The plugin impl's forward over one of setup's layers, as vLLM calls it: metadata
    with host query starts / sequence lengths, the new tokens' slots and the block table."""
    from oscar_amd.backend import OscarAttentionBackendImpl

    c = CONFIG
    d, hq, hk = c["d"], c["hq"], c["hk"]
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = d, hq, hk, setup.scale
    impl.key_cache = impl.value_cache = None
    os.environ.setdefault("OSCAR_ASCEND_VERBOSE", "0")
    impl._oscar_setup()
    kc, vc, (sk, sv, own) = setup.layers[layer_idx]
    layer = _Layer()
    layer._oscar_rots = (setup.rk, setup.rv)
    impl._set_caches((kc, vc))
    # the layer's window arena as bench's history writes left it
    layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner = sk, sv, own
    layer._oscar_stage_rows = own.shape[0]
    layer._oscar_stage_ready = impl._oscar_stage_ready = True
    impl.stage_block = c["block_size"]
    impl.sink_eff = setup.sink_eff
    # what cache initialization does in serving (integration.initialize_layers): the
    # stream's scratch and the transient workspaces at the sizes the batch limits give
    from oscar_amd import integration

    integration.reserve_device_scratch([impl], [(kc, vc)], max_tokens=setup.q.shape[0],
                                       max_len=max(setup.seqs), max_seqs=len(setup.seqs))
    md = _Meta()
    md.num_actual_tokens = setup.q.shape[0]
    md.slot_mapping = setup.slots
    md.query_start_loc_cpu = torch.tensor(setup.qsl, dtype=torch.int32)
    md.seq_lens_list = list(setup.seqs)
    md.block_tables = setup.bt
    q = setup.q.view(setup.q.shape[0], -1)
    k = setup.k_new.view(setup.k_new.shape[0], -1)
    v = setup.v_new.view(setup.v_new.shape[0], -1)
    out = torch.empty_like(q)
    return lambda: impl.forward(layer, q, k, v, (kc, vc), md, output=out)


def compare_calls_ms(fn, repeats=6):
    """delivery/benchmark_utils.py:9-70 for one variant: device-synchronised calls, the
    first call reported apart (first-use work), then `repeats` warm samples; median."""
    def measure():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    first = measure()
    warm = [measure() for _ in range(repeats)]
    return {"first_call_ms": first, "median_ms": float(np.median(warm)), "samples_ms": warm}


# tools/benchmark_streaming.py:16-20: (name, histories, query tokens per request), plus the
# config-5 batch in one call (the continuation, 16 decodes over 8192 tokens, a 2048-token
# history-free prefill)
FORWARD_CASES = (("mtp", [24579], 4), ("concurrent", [24579] * 8, 4), ("prefill", [15360], 9256),
                 ("config5_batched", [15360] + [8192] * 16 + [0], [9256] + [1] * 16 + [2048]))


def forward_timings(dev):
    """impl.forward per call at the reference's three bench cases (its scope: one layer's
    full forward incl. write, window and rotations), host-timed around device syncs."""
    res = {}
    for name, histories, count in FORWARD_CASES:
        setup = Setup(dev, histories, count, True, layers=1, seed=20261210)
        call = forward_call(setup)
        res[name] = compare_calls_ms(call)
        # back to back as a serving loop calls it (no synchronisation between calls):
        # the per-call rate once host work and device work overlap
        reps = 50 if name in ("mtp", "concurrent") else 5
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            call()
        torch.cuda.synchronize()
        res[name]["pipelined_ms"] = (time.perf_counter() - t0) * 1e3 / reps
        log(f"forward {name}: first {res[name]['first_call_ms']:.3f} ms, warm median "
            f"{res[name]['median_ms'] * 1e3:.1f} us, back to back {res[name]['pipelined_ms'] * 1e3:.1f} us/call")
        del setup, call
        torch.cuda.empty_cache()
    return res


def copy_ceiling_gbs(dev, mib=1024):
    """Device-to-device copy rate (read + write bytes / time) of a 1 GiB buffer."""
    src = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ms = event_ms(lambda r: dst.copy_(src), reps=5, warm=1)
    del src, dst
    torch.cuda.empty_cache()
    return 2 * (mib << 20) / (ms * 1e-3) / 1e9


def cpu_baseline(setup, budget_s=25.0, max_cores=16, cores=None):
    """The NumPy oracle of the same layer step (write 32 tokens + window, attention over
    8 x 24580 keys, inverse rotation) on this host: the first call is excluded, then
    warm samples until about budget_s of CPU work (at least 3), median reported."""
    from threadpoolctl import threadpool_limits

    from oracle import backend as ob
    from oracle.store import Staging

    if cores is None:
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
        cores = min(cores, max_cores)  # the one-GPU share of the host
    c = CONFIG
    kc, vc, (sk, sv, owner) = setup.layers[1]
    layer = ob.OracleLayer(k8=kc.view(torch.uint8).cpu().numpy(), v8=vc.view(torch.uint8).cpu().numpy(),
                           rk=setup.rk.cpu().numpy(), rv=setup.rv.cpu().numpy(), hq=c["hq"], hk=c["hk"],
                           d=c["d"], scale=setup.scale, sink_tokens=c["sink_tokens"],
                           recent_tokens=c["recent_tokens"], staging_tokens=c["staging_tokens"])
    st = Staging(c["block_size"], c["hk"], c["d"], c["sink_tokens"], c["recent_tokens"],
                 c["staging_tokens"])
    st.stage_k, st.stage_v, st.owner = sk.cpu().numpy(), sv.cpu().numpy(), owner.cpu().numpy()
    layer.staging = st
    q = setup.q.float().cpu().numpy()
    k = setup.k_new.float().cpu().numpy()
    v = setup.v_new.float().cpu().numpy()
    slots = setup.slots.cpu().numpy()
    bt = setup.bt.cpu().numpy()
    samples = []
    with threadpool_limits(limits=cores):
        start = time.perf_counter()
        while len(samples) < 4 or (time.perf_counter() - start < budget_s and len(samples) < 12):
            t0 = time.perf_counter()
            # the step rewrites the same 32 slots with the same tokens: repeat calls are identical
            ob.forward(layer, q, k, v, slots, setup.qsl, setup.seqs, bt)
            samples.append(time.perf_counter() - t0)
    warm = samples[1:]
    t = float(np.median(warm))
    kv_tokens = sum(setup.seqs)
    return {"value": kv_tokens / t, "unit": "KV-tokens/s", "cores": cores, "kind": "port",
            "sample": f"one full layer step of the headline workload (8 x {c['history']}+{c['q_len']} "
                      f"MTP: write + window + attention + inverse rotation) by the NumPy oracle; "
                      f"median of {len(warm)} warm samples (first call excluded), {t:.2f} s each"}


def measured_traffic():
    """HBM bytes per attn_main launch from the committed counter summary, or None."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes "):
            return float(line.split()[1])
    return None


def profile_main(setup, reps=3, copy_mib=1024):
    """Workload for the rocprofv3 counter passes: attn_main alone over the 16 layer
    caches, then two device copies of copy_mib MiB that calibrate FETCH/WRITE_SIZE: the
    runtime's blit copy and torch's vectorized elementwise kernel (16-byte lane loads
    and stores, the access width attn_main uses)."""
    for layer in range(LAYERS):  # one full step per layer: rotated q / k / v and the window
        setup.step(layer)
    torch.cuda.synchronize()
    for r in range(reps):
        for layer in range(LAYERS):
            setup.attention(layer, phases=1)
        torch.cuda.synchronize()
        log(f"attn_main pass {r + 1}/{reps} done")
    src = torch.ones(copy_mib << 18, dtype=torch.float32, device=setup.dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()
    log(f"calibration copies of {copy_mib} MiB done")


def pmc_summary(fetch_csv, write_csv, kernel="attn_main_kernel", copy_mib=1024):
    """HBM bytes per attn_main launch from the two counter passes, each scaled by what
    the same counter reads for the elementwise calibration copy (copy_mib MiB read and
    copy_mib MiB written); the blit copy's reading is reported beside it."""
    import csv

    def per_dispatch(path, counter):
        vals = {}
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                key = (row["Kernel_Name"], row["Dispatch_Id"])
                vals[key] = vals.get(key, 0.0) + float(row["Counter_Value"])
        return vals

    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        vals = per_dispatch(path, counter)
        main = [v for (name, _), v in vals.items() if kernel in name]
        ew = [v for (name, _), v in vals.items() if "MulFunctor" in name]
        blit = [v for (name, _), v in vals.items() if "copyBuffer" in name]
        if not main or not ew:
            raise SystemExit(f"{path}: no {kernel} or calibration dispatches with {counter}")
        scale = (copy_mib << 10) / max(ew)
        kib_main = float(np.median(main))
        out[counter] = {"kib_per_dispatch_raw": kib_main, "calib_elementwise_kib_raw": max(ew),
                        "calib_blit_kib_raw": max(blit) if blit else float("nan"),
                        "scale": scale, "bytes_per_dispatch": kib_main * scale * 1024,
                        "dispatches": len(main)}
    out["traffic_bytes"] = out["FETCH_SIZE"]["bytes_per_dispatch"] + out["WRITE_SIZE"]["bytes_per_dispatch"]
    return out


def rdreq_summary(rdreq_csv, kernel="attn_main_kernel"):
    """Read bytes per launch from the TCC/EA read-request counters by size (32, 64 and
    128 B), unscaled, with the same figure for the elementwise calibration copy: a
    cross-check of the scaled FETCH_SIZE (whose formula counts 128-byte requests as
    64 bytes on this part)."""
    import csv

    per = {}
    with open(rdreq_csv, newline="") as f:
        for row in csv.DictReader(f):
            key = (row["Kernel_Name"], row["Dispatch_Id"])
            per.setdefault(key, {})[row["Counter_Name"]] = float(row["Counter_Value"])

    def nbytes(v):
        return (v.get("TCC_EA0_RDREQ_128B_sum", 0) * 128 + v.get("TCC_EA0_RDREQ_64B_sum", 0) * 64
                + v.get("TCC_EA0_RDREQ_32B_sum", 0) * 32)

    main = [nbytes(v) for (name, _), v in per.items() if kernel in name]
    ew = [nbytes(v) for (name, _), v in per.items() if "MulFunctor" in name]
    n128 = [v.get("TCC_EA0_RDREQ_128B_sum", 0) for (name, _), v in per.items() if kernel in name]
    return {"read_bytes_per_dispatch": float(np.median(main)), "requests_128B_per_dispatch": float(np.median(n128)),
            "calib_elementwise_read_bytes": max(ew), "dispatches": len(main)}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-forward", action="store_true", help="skip the impl.forward timings")
    ap.add_argument("--config", default="4a", choices=["4a", "2", "3", "4b", "5"],
                    help="4a (default, the headline metric); 2 store; 3 single-request MTP; "
                         "4b 64 cache-only decodes; 5 continuation prefill")
    ap.add_argument("--clip", action="store_true",
                    help="the step's write with the serve defaults' sort clip (K 0.96, V 0.92; "
                         "delivery/serve_oscar.sh:32-33) instead of the library default (off)")
    ap.add_argument("--profile-main", action="store_true",
                    help="only run attn_main over the layer caches plus a calibration copy "
                         "(the workload of the rocprofv3 --pmc passes)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="FETCH_CSV WRITE_CSV [RDREQ_CSV]: turn the counter-collection CSVs into "
                         + str(TRAFFIC_FILE))
    args = ap.parse_args(argv)
    if args.clip:
        CONFIG.update(k_clip=0.96, v_clip=0.92)
    if args.pmc_summary:
        if len(args.pmc_summary) not in (2, 3):
            ap.error("--pmc-summary takes FETCH_CSV WRITE_CSV [RDREQ_CSV]")
        res = pmc_summary(*args.pmc_summary[:2])
        lines = [f"# attn_main_kernel<256>, config 4a (8 x 24576 + 4 MTP), HBM bytes per launch",
                 "# from rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE passes over",
                 "#   python bench.py --profile-main",
                 "# each scaled by the same counter's reading for a 1 GiB elementwise device copy"]
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            for k, v in res[counter].items():
                lines.append(f"{counter}.{k} {v}")
        lines.append(f"traffic_bytes {res['traffic_bytes']}")
        if len(args.pmc_summary) == 3:
            lines += ["# cross-check: rocprofv3 --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum",
                      "#   TCC_EA0_RDREQ_64B_sum TCC_EA0_RDREQ_128B_sum (same workload), unscaled"]
            for k, v in rdreq_summary(args.pmc_summary[2]).items():
                lines.append(f"RDREQ.{k} {v}")
        TRAFFIC_FILE.write_text("\n".join(lines) + "\n")
        print(TRAFFIC_FILE.read_text(), end="")
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this path runs on one GPU per TP rank "
              "(Hq=6, Hk=1 shard); multi-GPU runs are not part of this build", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from oscar_amd import _lib

    _lib.load()
    dev = torch.device("cuda", 0)
    if args.config != "4a":
        if args.config == "2":
            rec = config_store(dev)
        elif args.config == "3":
            rec = config_decode(dev, "config 3: 1 x (24576 INT2 history + 4-token MTP)", [24576], 4,
                                True, LAYERS, args.steps, args.warmup)
        elif args.config == "4b":
            hist = np.random.default_rng(20261204).integers(1024, 32769, 64).tolist()
            rec = config_decode(dev, "config 4b: 64 cache-only 1-token decodes, history U[1024, 32768]",
                                hist, 1, False, 4, args.steps, args.warmup)
        else:
            rec = config_prefill(dev)
        print(json.dumps(rec), flush=True)
        return 0
    log("building 16 layer caches (history store)")
    setup = Setup(dev)
    if args.profile_main:
        profile_main(setup)
        return 0
    staged = setup.staged_counts()
    b_main, b_op = setup.algorithmic_bytes(staged)
    log(f"staged history tokens per request: {staged}; B_main={b_main} B_op={b_op}")
    ms_step, steps, extra = time_graph(setup, args.steps, args.warmup)
    log(f"step {ms_step * 1e3:.2f} us ({steps} steps); 5 more replays: "
        + " ".join(f"{x * 1e3:.2f}" for x in extra) + " us")
    med_ms, mean_ms = time_main_kernel(setup)
    log(f"attn_main median {med_ms * 1e3:.2f} us mean {mean_ms * 1e3:.2f} us")
    achieved = b_main / (med_ms * 1e-3) / 1e9
    c = CONFIG
    kv_tokens = sum(setup.seqs)
    traffic = measured_traffic()
    ceiling = copy_ceiling_gbs(dev)
    log(f"device copy ceiling {ceiling:.0f} GB/s")
    rec = {
        "metric": "INT2-KV attention tokens/s + HBM GB/s (% peak), 8x24K MTP, one MI355X",
        "value": kv_tokens / (ms_step * 1e-3),
        "unit": "KV-tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2-kv/bf16",
        "data": "synthetic",
        "config": {"workload": "config 4a: 8 x (24576 INT2 history + 4-token MTP), one FULL layer "
                               "step (write + window + split-K attention + inverse rotation), "
                               "16 layer caches cycled",
                   "requests": c["requests"], "history": c["history"], "q_len": c["q_len"],
                   "hq": c["hq"], "hk": c["hk"], "head_dim": c["d"], "block_size": c["block_size"],
                   "layers_cycled": LAYERS, "staged_per_request": staged,
                   "clip": [c["k_clip"], c["v_clip"]]},
        "roofline": {"bound": "hbm", "kernel": "attn_main_kernel<256>", "achieved": achieved,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                     "algorithmic_bytes": b_main, "kernel_us": med_ms * 1e3,
                     "traffic": traffic,
                     "traffic_source": "from profile: " + str(TRAFFIC_FILE.relative_to(TRAFFIC_FILE.parents[1]))
                                       + " (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes)",
                     "physical_gbs": None if traffic is None else traffic / (med_ms * 1e-3) / 1e9,
                     "copy_ceiling_gbs": ceiling},
        "ms_per_step_replays": extra,
    }
    if not args.no_forward:
        log("impl.forward per call at the reference's bench cases")
        fw = forward_timings(dev)
        rec["forward_us"] = {k: v["median_ms"] * 1e3 for k, v in fw.items()}
        rec["forward_back_to_back_us"] = {k: v["pipelined_ms"] * 1e3 for k, v in fw.items()}
        rec["forward_first_call_ms"] = {k: v["first_call_ms"] for k, v in fw.items()}
    if not args.no_cpu:
        log("cpu baseline (NumPy oracle, one layer step)")
        rec["cpu_baseline"] = cpu_baseline(setup)
        log("cpu baseline at 2 threads (the reference tools' setting)")
        two = cpu_baseline(setup, budget_s=12.0, cores=2)
        rec["cpu_baseline_2threads"] = {k: two[k] for k in ("value", "unit", "cores", "kind")}
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
