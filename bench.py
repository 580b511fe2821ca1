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
              sink_tokens=64, recent_tokens=256, staging_tokens=8192)


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
    """16 layers of packed caches + staging arenas, and the step's static inputs."""

    def __init__(self, dev):
        from oscar_amd import ops
        from oscar_amd._lib import STAGE_INVALIDATE, STAGE_WRITE

        c = CONFIG
        B, L, n, hq, hk, d, bs = (c["requests"], c["history"], c["q_len"], c["hq"], c["hk"],
                                  c["d"], c["block_size"])
        self.dev = dev
        gen = torch.Generator(device=dev).manual_seed(20261201)
        pages = math.ceil((L + n) / bs)
        self.nb = B * pages
        self.bt = torch.randperm(self.nb, generator=gen, device=dev).view(B, pages).to(torch.int32)
        self.rk = hadamard_rotation(d, gen, dev)
        self.rv = hadamard_rotation(d, gen, dev).flip(0).contiguous()
        self.scale = d ** -0.5
        bs_ = bs
        self.sink_eff = (c["sink_tokens"] // bs_) * bs_
        rows = max(math.ceil(c["staging_tokens"] / bs_),
                   self.sink_eff // bs_ + math.ceil(c["recent_tokens"] / bs_) + 1 + 2)
        recent = c["recent_tokens"]
        pos = torch.arange(L, device=dev)
        hist_slots = (self.bt[:, (pos // bs)].long() * bs + pos % bs)        # [B, L]
        hist_k = outlier_kv(B * L, hk, d, gen, dev).view(B, L, hk, d)
        hist_v = outlier_kv(B * L, hk, d, gen, dev).view(B, L, hk, d)
        body, tail = slice(0, L - recent), slice(L - recent, L)
        qsl_t = torch.arange(0, B * recent + 1, recent, dtype=torch.int32, device=dev)
        seq_t = torch.full((B,), L, dtype=torch.int32, device=dev)
        self.layers = []
        for layer in range(LAYERS):
            kc = torch.zeros(self.nb, bs, hk, d, dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            stage = (torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                     torch.zeros(rows, bs, hk, d, dtype=torch.float32, device=dev),
                     torch.full((rows, bs), -1, dtype=torch.int64, device=dev))
            # standalone KV update of the prefix (tags nothing), then the window write
            ops.store(hist_k[:, body].reshape(-1, hk, d), hist_v[:, body].reshape(-1, hk, d), kc, vc,
                      hist_slots[:, body].reshape(-1), head_dim=d, rk=self.rk, rv=self.rv,
                      stage=stage, stage_mode=STAGE_INVALIDATE)
            ops.store(hist_k[:, tail].reshape(-1, hk, d), hist_v[:, tail].reshape(-1, hk, d), kc, vc,
                      hist_slots[:, tail].reshape(-1), head_dim=d, rk=self.rk, rv=self.rv,
                      stage=stage, stage_mode=STAGE_WRITE, qsl_dev=qsl_t, seqs_dev=seq_t,
                      num_reqs=B, recent_tokens=recent, sink_tokens_eff=self.sink_eff)
            self.layers.append((kc, vc, stage))
        del hist_k, hist_v
        torch.cuda.synchronize()
        # step inputs: 4 new tokens per request at positions L..L+3
        self.q = torch.randn(B * n, hq, d, generator=gen, device=dev).bfloat16()
        self.k_new = outlier_kv(B * n, hk, d, gen, dev)
        self.v_new = outlier_kv(B * n, hk, d, gen, dev)
        npos = torch.arange(L, L + n, device=dev)
        self.slots = (self.bt[:, npos // bs].long() * bs + npos % bs).reshape(-1).contiguous()
        self.qsl = [i * n for i in range(B + 1)]
        self.seqs = [L + n] * B
        self.qsl_dev = torch.tensor(self.qsl, dtype=torch.int32, device=dev)
        self.seq_dev = torch.tensor(self.seqs, dtype=torch.int32, device=dev)
        self.q_rot = torch.empty_like(self.q)
        self.k_rot = torch.empty_like(self.k_new)
        self.v_rot = torch.empty_like(self.v_new)
        self.out_rot = torch.zeros(B * n, hq, d, dtype=torch.float32, device=dev)
        self.lse = torch.zeros(B * n, hq, dtype=torch.float32, device=dev)
        self.out = torch.empty(B * n, hq, d, dtype=torch.bfloat16, device=dev)
        self.plan = ops.plan_decode(self.qsl, self.seqs, has_new=True, num_kv_heads=hk,
                                    group=hq // hk, head_dim=d, device=dev)

    def step(self, layer, phases=0):
        from oscar_amd import ops
        from oscar_amd._lib import STAGE_WRITE

        c = CONFIG
        kc, vc, stage = self.layers[layer]
        ops.store(self.k_new, self.v_new, kc, vc, self.slots, head_dim=c["d"], rk=self.rk,
                  rv=self.rv, stage=stage, stage_mode=STAGE_WRITE, qsl_dev=self.qsl_dev,
                  seqs_dev=self.seq_dev, num_reqs=c["requests"], recent_tokens=c["recent_tokens"],
                  sink_tokens_eff=self.sink_eff, query=self.q, query_rot=self.q_rot,
                  key_rot=self.k_rot, value_rot=self.v_rot)
        self.attention(layer)
        ops.rotate(self.out_rot, self.rv, transpose=True, out_dtype=torch.bfloat16, out=self.out)

    def attention(self, layer, phases=0):
        from oscar_amd import ops

        kc, vc, stage = self.layers[layer]
        ops.attention_decode(self.q_rot, self.k_rot, self.v_rot, kc, vc, self.bt, self.plan,
                             self.scale, stage, head_dim=CONFIG["d"], out_rot=self.out_rot,
                             lse=self.lse, phases=phases)

    def staged_counts(self):
        """Per-request count of history tokens whose owner tag selects the FP32 window."""
        c = CONFIG
        _, _, (_, _, owner) = self.layers[0]
        own = owner.cpu().numpy()
        bt = self.bt.cpu().numpy().astype(np.int64)
        bs, L = c["block_size"], c["history"]
        pos = np.arange(L)
        counts = []
        for r in range(c["requests"]):
            blk = bt[r, pos // bs]
            counts.append(int((own[blk % own.shape[0], pos % bs] == blk).sum()))
        return counts


def algorithmic_bytes(staged):
    """Unique bytes the attention pass must touch (history codes+meta, staged FP32
    window, page-table entries, q, current k/v, owner tags) and the op's outputs."""
    c = CONFIG
    L, n, hq, hk, d, bs = c["history"], c["q_len"], c["hq"], c["hk"], c["d"], c["block_size"]
    per_req = [136 * L + 2048 * s + 4 * math.ceil(L / bs) + 2 * n * hq * d + 4 * n * hk * d
               for s in staged]
    owner = 8 * math.ceil(c["staging_tokens"] / bs) * bs
    b_main = sum(per_req) + owner
    b_out = c["requests"] * n * hq * (2 * d + 4)
    return b_main, b_main + b_out


def time_graph(setup, steps, warmup):
    """Whole-step time: a HIP graph of LAYERS layer steps replayed steps/LAYERS times."""
    for i in range(max(warmup, LAYERS)):
        setup.step(i % LAYERS)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for layer in range(LAYERS):
                setup.step(layer)
    torch.cuda.current_stream().wait_stream(stream)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // LAYERS)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    wall = t0.elapsed_time(t1)
    return wall / (reps * LAYERS), reps * LAYERS


def time_main_kernel(setup, reps=8):
    """Average duration of attn_main alone: a spin kernel keeps the stream busy while the
    host enqueues event -> kernel -> event, so the pair brackets only the kernel."""
    durs = []
    for r in range(reps):
        for layer in range(LAYERS):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(2_000_000)
            e0.record()
            setup.attention(layer, phases=1)
            e1.record()
            e1.synchronize()
            durs.append(e0.elapsed_time(e1))
    durs = np.array(durs[LAYERS:])  # first pass over the layers is warm-up
    return float(np.median(durs)), float(durs.mean())


def cpu_baseline(setup, budget_s=25.0, max_cores=16):
    """The NumPy oracle of the same layer step (write 32 tokens + window, attention over
    8 x 24580 keys, inverse rotation) on this host: the first call is excluded, then
    warm samples until about budget_s of CPU work (at least 3), median reported."""
    from threadpoolctl import threadpool_limits

    from oracle import backend as ob
    from oracle.store import Staging

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


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--profile-main", action="store_true",
                    help="only run attn_main over the layer caches plus a calibration copy "
                         "(the workload of the rocprofv3 --pmc passes)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn the two counter-collection CSVs into " + str(TRAFFIC_FILE))
    args = ap.parse_args(argv)
    if args.pmc_summary:
        res = pmc_summary(*args.pmc_summary)
        lines = [f"# attn_main_kernel<256>, config 4a (8 x 24576 + 4 MTP), HBM bytes per launch",
                 "# from rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE passes over",
                 "#   python bench.py --profile-main",
                 "# each scaled by the same counter's reading for a 1 GiB elementwise device copy"]
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            for k, v in res[counter].items():
                lines.append(f"{counter}.{k} {v}")
        lines.append(f"traffic_bytes {res['traffic_bytes']}")
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
    log("building 16 layer caches (history store)")
    setup = Setup(dev)
    if args.profile_main:
        profile_main(setup)
        return 0
    staged = setup.staged_counts()
    b_main, b_op = algorithmic_bytes(staged)
    log(f"staged history tokens per request: {staged}; B_main={b_main} B_op={b_op}")
    ms_step, steps = time_graph(setup, args.steps, args.warmup)
    log(f"step {ms_step * 1e3:.2f} us ({steps} steps)")
    med_ms, mean_ms = time_main_kernel(setup)
    log(f"attn_main median {med_ms * 1e3:.2f} us mean {mean_ms * 1e3:.2f} us")
    achieved = b_main / (med_ms * 1e-3) / 1e9
    c = CONFIG
    kv_tokens = sum(setup.seqs)
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
                   "layers_cycled": LAYERS, "staged_per_request": staged},
        "roofline": {"bound": "hbm", "kernel": "attn_main_kernel<256>", "achieved": achieved,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                     "algorithmic_bytes": b_main, "kernel_us": med_ms * 1e3,
                     "traffic": measured_traffic()},
    }
    if not args.no_cpu:
        log("cpu baseline (NumPy oracle, one layer step)")
        rec["cpu_baseline"] = cpu_baseline(setup)
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
