"""CPU emulation of attn_main_kernel's address arithmetic over random plans.

Every global access the decode kernel makes is restated here from the kernel's own
index expressions (attn_decode.hip: item record, page ids, tile loads of the fast and
slow paths, owner tags, staged FP32 rows, current-chunk rows, queries, partials) and
checked against the extent of the buffer it reads or writes, for plans produced by
oscar_attn_plan_v1 over random batches and cache geometries -- including block
tables holding ids outside the cache, which the kernel clamps.  A change to the
planner or to the kernel's indexing that lets an access leave its buffer fails here,
on the CPU, before any GPU run.
"""
import ctypes as C

import numpy as np
import pytest

from oscar_amd import _lib

TILE = 32
WAVES = 8
MAX_TILES = 8192 // TILE


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from oscar_amd import build

        build.build()
    return _lib.load()


def make_plan(lib, qsl, seqs, has_new, hk, group, d, target, window):
    n = len(seqs)
    qa, sa = (C.c_int32 * (n + 1))(*qsl), (C.c_int32 * max(n, 1))(*seqs)
    p = _lib.Plan()
    lib.oscar_attn_plan_v1(qa, sa, n, int(has_new), hk, group, d, 8192, target, *window,
                           None, 0, None, 0, C.byref(p))
    items = (C.c_int32 * max(p.num_items * 8, 1))()
    groups = (C.c_int32 * max(p.num_groups * 8, 1))()
    cnt = lib.oscar_attn_plan_v1(qa, sa, n, int(has_new), hk, group, d, 8192, target, *window,
                                 items, p.num_items, groups, p.num_groups, C.byref(p))
    assert cnt == p.num_items
    return np.array(items[: cnt * 8], np.int64).reshape(-1, 8)


class Extent:
    """Collects [lo, hi) byte ranges per buffer and checks them against the sizes."""

    def __init__(self, sizes):
        self.sizes, self.bad = sizes, []

    def access(self, buf, lo, nbytes, what):
        lo = np.asarray(lo, np.int64)
        hi = lo + nbytes
        out = (lo < 0) | (hi > self.sizes[buf])
        if out.any():
            self.bad.append((buf, what, int(lo[out].min()), int(hi[out].max()), self.sizes[buf]))


def emulate(items, g):
    """The kernel's accesses for every item (vectorised over lanes / tokens)."""
    D, hk, bs, G = g["D"], g["hk"], g["bs"], g["group"]
    ks0, ks1, ks2 = g["k_stride"]
    vs0, vs1, vs2 = g["v_stride"]
    rows, nb = g["rows"], g["num_blocks"]
    ext = Extent(g["sizes"])
    m = np.arange(32)[:, None]          # token of a tile (lane % 32)
    half = np.arange(2)[None, :]        # lane half g
    for idx, it in enumerate(items):
        ext.access("items", idx * 8 * 4, 32, "item record")
        req, kvh, nq = it[0], it[1] & 0xFFFF, it[1] >> 16
        first, stride, count, part, qa, seq = it[2:8]
        stride, off = stride & 0xFFF, stride >> 12
        hist = seq - nq - off if g["has_new"] else seq
        cur0 = qa - off
        nrows = nq * G
        # the kernel's rule: a record outside the plan's contract poisons its partial
        if (req < 0 or req >= g["num_reqs"] or kvh >= hk or nq < 1 or nrows > 32 or hist < 0 or off < 0
                or cur0 < 0
                or qa + nq > g["num_tokens"] or first < 0 or stride < 1 or count < 0 or count > MAX_TILES
                or (count > 0 and (first + stride * (count - 1)) * TILE >= seq)):
            ext.access("part_lse", part * 32 * 4, 32 * 4, "poisoned lse")
            continue
        t0 = (first + stride * np.arange(count)) * TILE
        # page ids (lane i of wave w: item tile w + 8 i), history tiles only
        hist_tiles = t0 < hist
        ext.access("table", (req * g["bt_stride"] + t0[hist_tiles] // bs) * 4, 4, "page id")
        blk = np.zeros(count, np.int64)
        raw = g["table"][req, t0[hist_tiles] // bs]
        blk[hist_tiles] = np.where((raw < 0) | (raw >= nb), 0, raw)  # in-kernel clamp
        seat = (blk % rows) * bs if g["staged"] else np.zeros(count, np.int64)
        off0 = np.where(hist_tiles, t0 % bs, 0)
        # queries: lane (row n, half g) reads D/2 elements of its row (clamped to row 0)
        n = np.minimum(np.arange(32), nrows - 1)
        qtok, qhead = qa + n // G, kvh * G + n % G
        ext.access("q", ((qtok * g["q_stride"] + qhead * D)[:, None] + half * (D // 2)) * 2, D, "query row")
        # fast / prologue tile loads: K codes + meta, V codes of tokens off0 + m of the
        # tile's block (placeholder: block 0, offsets 0..31)
        for j in list(range(count)) + [count]:
            b, o = (blk[j], off0[j]) if j < count else (0, 0)
            kslot = kvh * ks2 + b * ks0 + (o + m) * ks1
            vslot = kvh * vs2 + b * vs0 + (o + m) * vs1
            ext.access("k", kslot + 32 + half * (D // 8), D // 8, "K codes")
            ext.access("k", kslot, 8, "meta")
            ext.access("v", vslot + half * (D // 8), D // 8, "V codes")
            if g["staged"] and j < count and t0[j] < hist:
                ext.access("owner", (seat[j] + off0[j] + m[:, 0]) * 8, 8, "owner tag")
                # slow path: staged FP32 rows of the tile's tokens (K and V)
                srow = ((seat[j] + off0[j] + m[:, 0]) * hk + kvh) * D
                ext.access("stage", srow * 4, D * 4, "staged row")
        # slow path: current-chunk rows (positions hist .. seq - 1 of the tiles)
        if g["has_new"]:
            pos = (t0[:, None] + m[:, 0][None, :]).ravel()
            cur = pos[(pos >= hist) & (pos < seq)]
            ext.access("kv_new", ((cur0 + cur - hist) * g["kv_stride"] + kvh * D) * 2, D * 2, "current row")
        ext.access("part_o", part * 32 * D * 4, 32 * D * 4, "item partial")
        ext.access("part_lse", part * 32 * 4, 32 * 4, "item lse")
    return ext.bad


@pytest.mark.parametrize("seed", range(12))
def test_decode_accesses_stay_in_their_buffers(lib, seed):
    rng = np.random.default_rng(31000 + seed)
    for _ in range(6):
        D = int(rng.choice([128, 256]))
        hk = int(rng.choice([1, 2]))
        group = int(rng.choice([1, 2, 3, 4, 6]))
        has_new = bool(rng.integers(2))
        bs = int(rng.choice([32, 64, 128, 256, 1536]))
        staged = bool(rng.integers(2))
        legacy = bool(rng.integers(2))
        nreq = int(rng.integers(1, 24))
        lens = rng.integers(0 if not has_new else 1, 32 // group + 1, nreq)
        lens[rng.random(nreq) < 0.2] *= 9                           # chunks cut into sub-requests
        if lens.sum() == 0:
            lens[0] = 1
        qsl = [0] + np.cumsum(lens).tolist()
        hist = rng.integers(0, 30000, nreq) * (rng.random(nreq) < 0.9)
        seqs = (hist + (lens if has_new else 0)).tolist()
        if not has_new:
            seqs = [max(s, 1) for s in seqs]
        target = int(rng.choice([1, 16, 256, 1024]))
        window = (int(rng.choice([0, 128])), int(rng.choice([0, 256, 2048])))
        items = make_plan(lib, qsl, seqs, has_new, hk, group, D, target, window)
        width = max(1, max(-(-(s - (l if has_new else 0)) // bs) for s, l in zip(seqs, lens)))
        width += int(rng.integers(0, 3))
        num_blocks = int(rng.integers(1, nreq * width + 2))
        table = rng.integers(0, num_blocks, (nreq, width))
        table[rng.random(table.shape) < 0.05] = -7                   # ids the kernel clamps
        table[rng.random(table.shape) < 0.05] = num_blocks + 11
        slot = 2 * D if legacy else D
        rows = int(rng.choice([4, 64]))
        N = qsl[-1]
        g = dict(D=D, hk=hk, bs=bs, group=group, has_new=has_new, staged=staged, rows=rows,
                 num_blocks=num_blocks, num_reqs=nreq, num_tokens=N, table=table, bt_stride=width,
                 k_stride=(bs * hk * slot, hk * slot, slot), v_stride=(bs * hk * slot, hk * slot, slot),
                 q_stride=hk * group * D, kv_stride=hk * D,
                 sizes=dict(items=len(items) * 32, table=table.size * 4,
                            k=num_blocks * bs * hk * slot, v=num_blocks * bs * hk * slot,
                            owner=rows * bs * 8, stage=rows * bs * hk * D * 4,
                            q=N * hk * group * D * 2, kv_new=N * hk * D * 2,
                            part_o=len(items) * 32 * D * 4, part_lse=len(items) * 32 * 4))
        bad = emulate(items, g)
        assert not bad, f"out-of-bounds accesses: {bad[:3]} (geometry {dict((k, g[k]) for k in ('D', 'hk', 'bs', 'group', 'has_new', 'rows', 'num_blocks'))})"


def test_emulation_reports_a_table_too_narrow_for_the_history(lib):
    """The emulation is sharp: with a block-table row narrower than the history (what
    the host-side table check rejects before any launch), the page-id reads past the
    row are reported."""
    D, bs, width = 256, 128, 16                       # 16 pages cover 2048 tokens
    seqs, qsl = [40000], [0, 4]
    items = make_plan(lib, qsl, seqs, True, 1, 6, D, 256, (0, 0))
    table = np.zeros((1, width), np.int64)
    g = dict(D=D, hk=1, bs=bs, group=6, has_new=True, staged=False, rows=64, num_blocks=width,
             num_reqs=1, num_tokens=4, table=np.zeros((1, 400), np.int64), bt_stride=width,
             k_stride=(bs * D, D, D), v_stride=(bs * D, D, D), q_stride=6 * D, kv_stride=D,
             sizes=dict(items=len(items) * 32, table=table.size * 4, k=width * bs * D, v=width * bs * D,
                        owner=64 * bs * 8, stage=64 * bs * D * 4, q=4 * 6 * D * 2, kv_new=4 * D * 2,
                        part_o=len(items) * 32 * D * 4, part_lse=len(items) * 32 * 4))
    bad = emulate(items, g)
    assert any(b[1] == "page id" for b in bad)
