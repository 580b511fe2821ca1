"""The C-ABI boundary on the CPU: exports, struct layout, host planner, argument checks.

Nothing here launches a kernel: the library is loaded and only its host-side
functions (planner, size queries, argument validation) are called.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oscar_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "oscar_amd.h"
TILE = 32


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from oscar_amd import build

        build.build()
    return _lib.load()


def header_functions() -> set:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(oscar_[a-z_0-9]+)\s*\(", text, flags=re.M))


def test_library_exports_every_header_symbol(lib):
    names = header_functions()
    assert len(names) == 17, names
    for name in names:
        assert hasattr(lib, name), name
    assert names == set(_lib.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T oscar_" in line}
    assert exported == names  # nothing undeclared leaks out
    assert lib.oscar_abi_version() == int(re.search(r"OSCAR_ABI_VERSION (\d+)", HEADER.read_text())[1])


STRUCTS = {
    "oscar_cache_v1": _lib.Cache, "oscar_staging_v1": _lib.Staging,
    "oscar_store_args_v1": _lib.StoreArgs, "oscar_rotate_args_v1": _lib.RotateArgs,
    "oscar_plan_v1": _lib.Plan, "oscar_attn_args_v1": _lib.AttnArgs,
    "oscar_prefill_args_v1": _lib.PrefillArgs, "oscar_step_args_v1": _lib.StepArgs,
}


def test_ctypes_structs_match_c_layout(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["return 0; }"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, py in STRUCTS.items():
        assert got[(cname, "size")] == C.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


# ------------------------------------------------------------------ planner
def plan(lib, qsl, seqs, has_new=True, hk=1, group=6, d=256, chunk=8192, target=256, window=(0, 0)):
    n = len(seqs)
    qa = (C.c_int32 * (n + 1))(*qsl)
    sa = (C.c_int32 * max(n, 1))(*seqs)
    p = _lib.Plan()
    cnt = lib.oscar_attn_plan_v1(qa, sa, n, int(has_new), hk, group, d, chunk, target, *window, None, 0,
                                 None, 0, C.byref(p))
    if cnt < 0:
        return cnt, None, None, p
    items = (C.c_int32 * max(p.num_items * 8, 1))()
    groups = (C.c_int32 * max(p.num_groups * 8, 1))()
    cnt = lib.oscar_attn_plan_v1(qa, sa, n, int(has_new), hk, group, d, chunk, target, *window, items,
                                 p.num_items, groups, p.num_groups, C.byref(p))
    assert cnt == p.num_items
    it = np.array(list(items)[:p.num_items * 8], np.int64).reshape(-1, 8)
    gr = np.array(list(groups)[:p.num_groups * 8], np.int64).reshape(-1, 8)
    return cnt, it, gr, p


def item_tiles(it):
    return it[2] + (it[3] & 0xFFF) * np.arange(it[4])


def sub_requests(qsl, seqs, has_new, group):
    """The planner's (sub-)requests: (request, first query token, queries, keys, offset
    in the chunk) for every cut of 32 // group query tokens of a non-empty request."""
    sub = 32 // group
    out = []
    for r, (a0, b0, s) in enumerate(zip(qsl, qsl[1:], seqs)):
        nq = b0 - a0
        for a in range(0, nq, sub):
            b = min(nq, a + sub)
            out.append((r, a0 + a, b - a, max(0, s - (nq - b)), a if has_new else 0))
    return out


PLAN_CASES = [
    ([0, 4, 7, 8, 10], [133, 1028, 4, 302], True, 1, 6),      # MTP, mixed lengths
    ([0] + [4 * i for i in range(1, 9)], [24580] * 8, True, 1, 6),
    ([0, 1, 1, 5, 10], [0, 257, 3, 263], False, 1, 6),        # cache-only, empty request
    ([0, 4, 6], [1025, 702], True, 2, 4),
    ([0] + list(range(1, 65)), [2048 + 37 * i for i in range(64)], False, 1, 6),
    ([0] + list(range(1, 65)), [1024 + 487 * i for i in range(64)], False, 1, 6),
    ([0, 40, 47, 48], [3040, 507, 9000], True, 1, 6),           # chunks of 240 and 42 rows
    ([0, 20, 37], [700, 4017], False, 2, 4),                    # cache-only, 80 and 68 rows
]


@pytest.mark.parametrize("window", [(0, 0), (128, 256), (0, 4096)])
@pytest.mark.parametrize("qsl,seqs,has_new,hk,group", PLAN_CASES)
def test_plan_covers_every_tile_once_and_respects_kernel_limits(lib, qsl, seqs, has_new, hk, group, window):
    check_plan(lib, qsl, seqs, has_new, hk, group, window, 256, 256)


def check_plan(lib, qsl, seqs, has_new, hk, group, window, target, d):
    """The plan's contract with the decode kernel: every key tile of every group in
    exactly one item, partial slots a permutation, item limits, group records."""
    cnt, items, groups, p = plan(lib, qsl, seqs, has_new, hk, group, d=d, target=target, window=window)
    assert cnt > 0
    assert sorted(items[:, 5].tolist()) == list(range(cnt))          # partial slots: a permutation
    assert p.partial_bytes == cnt * 32 * (d + 1) * 4
    subs = {(r, qa): (nq, seq, off) for r, qa, nq, seq, off in sub_requests(qsl, seqs, has_new, group)}
    ngroups = hk * len(subs)
    # within the target, unless the groups need more: an item holds at most 256 tiles
    floor = hk * sum(max(1, -(-(-(-seq // TILE)) // 256)) for nq, seq, off in subs.values())
    assert cnt <= max(target, floor)
    for it in items:
        req, kvh, nq, first, stride, count, part, qa, seq = (it[0], it[1] & 0xFFFF, it[1] >> 16, *it[2:8])
        stride, off = stride & 0xFFF, stride >> 12
        assert subs[(req, qa)] == (nq, seq, off)
        assert 0 <= kvh < hk and nq * group <= 32
        assert 0 <= first and stride >= 1 and (count > 0 or (first == 0 and stride == 1))
        assert count <= 8192 // TILE
        assert count == 0 or (first + stride * (count - 1)) * TILE < seq   # no tile past the end
    # per group: every tile of [0, ceil(seq / 32)) exactly once, slots contiguous
    for req, kvh, first_slot, nslots, qa, nq, z0, z1 in groups:
        assert subs[(req, qa)][0] == nq and z0 == z1 == 0
        rows = items[(items[:, 0] == req) & ((items[:, 1] & 0xFFFF) == kvh) & (items[:, 6] == qa)]
        assert sorted(rows[:, 5].tolist()) == list(range(first_slot, first_slot + nslots))
        cover = np.zeros((subs[(req, qa)][1] + TILE - 1) // TILE, np.int64)
        for it in rows:
            np.add.at(cover, item_tiles(it), 1)
        assert (cover == 1).all()
    assert len(groups) == ngroups
    assert p.max_group_items == groups[:, 3].max()


@pytest.mark.parametrize("seed", range(8))
def test_plan_random_requests_cover_every_tile_once(lib, seed):
    """Seeded random batches: request counts, query lengths (MTP, decode, cache-only,
    empty), history lengths from 0 to 40K, window hints, targets, Hk and head dims."""
    rng = np.random.default_rng(9000 + seed)
    for _ in range(25):
        hk = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 3, 4, 6, 8]))
        has_new = bool(rng.integers(2))
        nreq = int(rng.integers(1, 40))
        lens = rng.integers(0 if not has_new else 1, 32 // group + 1, nreq)
        lens[rng.random(nreq) < 0.15] *= 7                          # more than 32 rows: sub-requests
        lens[rng.random(nreq) < 0.1] = 0                            # empty requests
        if lens.sum() == 0:
            lens[0] = 1
        qsl = [0] + np.cumsum(lens).tolist()
        hist = rng.integers(0, 40000, nreq) * (rng.random(nreq) < 0.9)
        seqs = (hist + (lens if has_new else 0)).tolist()
        if not has_new:
            seqs = [max(s, 1) for s in seqs]
        window = tuple(int(v) for v in rng.choice([0, 128, 512], 1).tolist() +
                       rng.choice([0, 256, 2048], 1).tolist())
        target = int(rng.choice([1, 16, 100, 256, 1024]))
        d = int(rng.choice([128, 256]))
        check_plan(lib, qsl, seqs, has_new, hk, group, window, target, d)


def test_plan_without_window_deals_history_evenly(lib):
    # no window hint: the history tiles of a group go round-robin to items within one
    # tile of each other; the one tile holding the current chunk goes to an item of its own
    _, items, _, _ = plan(lib, [0] + [4 * i for i in range(1, 9)], [24580] * 8)
    for r in range(8):
        rows = items[items[:, 0] == r]
        hist_rows = [it for it in rows if item_tiles(it).max() < 768]
        cur_rows = [it for it in rows if 768 in item_tiles(it)]
        assert len(cur_rows) == 1 and cur_rows[0][4] == 1
        sizes = [it[4] for it in hist_rows]
        assert len(hist_rows) + 1 == len(rows) and max(sizes) - min(sizes) <= 1
    assert len(items) <= 256 and items[:, 4].max() <= 25


def test_plan_puts_the_expected_window_in_items_of_its_own(lib):
    # 8 x (24576 + 4 MTP), recent window 256: tiles >= (24580 - 256) // 32 = 760 are
    # expected FP32 (or current) tiles; sink 128 -> tiles 0..3
    _, items, _, _ = plan(lib, [0] + [4 * i for i in range(1, 9)], [24580] * 8, window=(128, 256))
    assert len(items) <= 256
    for it in items:
        t = item_tiles(it)
        kinds = {"sink" if x < 4 else ("tail" if x >= 760 else "body") for x in t}
        assert len(kinds) == 1, (it, kinds)
    window_items = [it for it in items if item_tiles(it).max() >= 760 or item_tiles(it).min() < 4]
    assert max(it[4] for it in window_items) >= 2          # several window tiles per item
    body = [it[4] for it in items if 4 <= item_tiles(it).min() and item_tiles(it).max() < 760]
    assert max(body) - min(body) <= 1


def test_plan_keeps_short_groups_whole(lib):
    # 64 cache-only requests: a 1024-token request is one item even with the hint
    # (its 9 window tiles are cheaper together than another item), long ones are split
    seqs = [1024 + 487 * i for i in range(64)]
    _, items, _, _ = plan(lib, list(range(65)), seqs, has_new=False, window=(0, 256))
    assert len(items) <= 256
    assert (items[:, 0] == 0).sum() == 1
    for r in (40, 63):
        rows = items[items[:, 0] == r]
        w0 = (seqs[r] - 256) // TILE
        tail = [it for it in rows if item_tiles(it).max() >= w0]
        assert all(item_tiles(it).min() >= w0 for it in tail)


@pytest.mark.parametrize("window", [(0, 0), (128, 256)])
def test_plan_larger_target_never_makes_items_larger(lib, window):
    seqs = [1024 + 487 * i for i in range(64)]
    prev = None
    for target in (64, 128, 256, 512, 1024):
        _, items, _, _ = plan(lib, list(range(65)), seqs, has_new=False, target=target, window=window)
        floor_items = sum(-(-s // (TILE * 256)) for s in seqs)   # at most 256 tiles per item
        assert len(items) <= max(target, floor_items)
        big = items[:, 4].max()
        assert prev is None or big <= prev
        prev = big


def test_plan_launch_order_interleaves_groups(lib):
    _, items, _, _ = plan(lib, [0] + [4 * i for i in range(1, 9)], [24580] * 8)
    # item p of every group before item p + 1 of any group
    assert items[:8, 0].tolist() == list(range(8))
    slot0 = {r: items[items[:, 0] == r][:, 5].min() for r in range(8)}
    pos = np.array([it[5] - slot0[it[0]] for it in items])
    assert (np.diff(pos) >= 0).all()


def test_plan_cuts_long_chunks_into_sub_requests(lib):
    # a continuation chunk of 12 tokens at 6 heads per KV head (72 rows): sub-requests of
    # 5, 5 and 2 queries, each its own group; their key ranges end at their last query
    cnt, items, groups, _ = plan(lib, [0, 12], [5012], has_new=True, group=6)
    assert groups[:, 4].tolist() == [0, 5, 10] and groups[:, 5].tolist() == [5, 5, 2]
    for qa, nq in ((0, 5), (5, 5), (10, 2)):
        rows = items[items[:, 6] == qa]
        assert (rows[:, 7] == 5000 + qa + nq).all() and ((rows[:, 3] >> 12) == qa).all()
        assert ((rows[:, 1] >> 16) == nq).all()


def test_plan_caps_items_per_group(lib):
    # one long request: at most 128 items (one load round of the merge's 8 waves x 16)
    # however large the target
    for seq, target in ((24580, 256), (100003, 1024), (40000, 4096)):
        cnt, items, groups, p = plan(lib, [0, 4], [seq], target=target)
        assert cnt == groups[0, 3] and cnt <= 128 and p.max_group_items == cnt
    # 8 requests of that length still take the whole target
    cnt, *_ = plan(lib, [0] + [4 * i for i in range(1, 9)], [24580] * 8, target=256)
    assert 200 < cnt <= 256


def test_plan_splits_long_history_across_items(lib):
    _, items, _, _ = plan(lib, [0, 4], [100003], target=256)
    assert len(items) > 64 and items[:, 4].max() * TILE <= 8192


def test_plan_rejects_bad_requests(lib):
    cnt, *_ = plan(lib, [0, 1], [100], group=33)            # 33 heads per KV head: no 32-row tile
    assert cnt == -22 and b"query heads" in lib.oscar_last_error()
    cnt, *_ = plan(lib, [0, 4], [3], has_new=True)          # sequence shorter than its chunk
    assert cnt == -22
    cnt, *_ = plan(lib, [0, 1], [10], d=96)
    assert cnt == -22 and b"head_dim" in lib.oscar_last_error()
    qa, sa = (C.c_int32 * 2)(0, 1), (C.c_int32 * 1)(100)
    p = _lib.Plan()
    small = (C.c_int32 * 16)()
    assert lib.oscar_attn_plan_v1(qa, sa, 1, 1, 1, 6, 256, 32, 64, 0, 0, small, 1, small, 2, C.byref(p)) == -28
    cnt, *_ = plan(lib, [0, 1], [10], window=(-1, 0))
    assert cnt == -22


def test_empty_plan(lib):
    cnt, items, groups, p = plan(lib, [0, 0, 0], [5, 7])
    assert cnt == 0 and p.num_groups == 0 and p.partial_bytes == 0


# ------------------------------------------------------------------ argument checks
def test_entry_points_reject_null_and_unsupported_args_without_touching_the_gpu(lib):
    assert lib.oscar_store_v1(None, None) == -22
    assert b"null" in lib.oscar_last_error()
    assert lib.oscar_rotate_v1(None, None) == -22
    assert lib.oscar_attn_decode_v1(None, None) == -22
    assert lib.oscar_attn_decode_static_v1(None, None) == -22
    assert lib.oscar_decode_write_v1(None, None, None) == -22
    assert lib.oscar_attn_prefill_v1(None, None) == -22
    r = _lib.RotateArgs(rows=4, head_dim=96, x=1, r=1, out=1)
    assert lib.oscar_rotate_v1(C.byref(r), None) == -22 and b"head_dim" in lib.oscar_last_error()
    r = _lib.RotateArgs(rows=0)
    assert lib.oscar_rotate_v1(C.byref(r), None) == 0  # nothing to do
    s = _lib.StoreArgs(num_tokens=3)
    s.cache.head_dim = 200
    assert lib.oscar_store_v1(C.byref(s), None) == -22
    s = _lib.StoreArgs(num_tokens=0)
    assert lib.oscar_store_v1(C.byref(s), None) == 0
    # <= 64 tokens: the column slices y [2][N][Hk][D] fp32
    assert lib.oscar_store_workspace_bytes_v1(10, 2, 256) == 2 * 10 * 2 * 256 * 4
    # larger: exact-pass totals, per-workgroup counts (2 x 1024) and lists (2 N Hk), int32,
    # 16-B padded + window flags [N] int32 + fp16 planes of R_k and R_v (8 D^2 bytes) +
    # column exponents and norms (16 D bytes)
    lists = ((2 + 2 * 1024 + 2 * 100 * 2) * 4 + 15) // 16 * 16
    assert lib.oscar_store_workspace_bytes_v1(100, 2, 256) == lists + 400 + 8 * 256 * 256 + 16 * 256


def decode_args(**kw):
    """Decode arguments that pass every host check before the launch (placeholder
    device addresses; the calls below are rejected before anything is launched)."""
    a = _lib.AttnArgs(q=0x10000, num_tokens=4, num_q_heads=6, q_stride_token=1536,
                      block_table=0x20000, block_table_stride=16, query_start_loc=0x30000,
                      seq_lens=0x40000, num_reqs=1, scale=0.0625, items=0x50000, num_items=4,
                      groups=0x60000, num_groups=1, workspace=0x70000, out_rot=0x80000,
                      lse=0x90000, q_dtype=_lib.OSCAR_BF16)
    a.cache.k, a.cache.v = 0x100000, 0x200000
    a.cache.num_blocks, a.cache.block_size, a.cache.num_kv_heads, a.cache.head_dim = 8, 128, 1, 256
    for i, st in enumerate((128 * 256, 256, 256)):
        a.cache.k_stride[i] = a.cache.v_stride[i] = st
    a.workspace_bytes = 4 * 32 * 257 * 4
    a.max_group_items = 4
    a.block_table_rows, a.block_table_cols = 1, 16
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_decode_rejects_a_table_with_missing_rows_or_columns(lib):
    """streaming_attention.py:48-50: the table needs a row per request and at least one
    column (its stride at least its width); checked before anything is launched."""
    for kw in (dict(block_table_rows=0), dict(block_table_cols=0), dict(block_table_cols=17),
               dict(num_reqs=2, block_table_rows=1)):
        a = decode_args(**kw)
        for entry in ("oscar_attn_decode_v1", "oscar_attn_decode_static_v1"):
            assert getattr(lib, entry)(C.byref(a), None) == -22, (kw, entry)
            assert b"Missing request block-table rows" in lib.oscar_last_error()
        assert lib.oscar_decode_write_v1(C.byref(_lib.StoreArgs(num_tokens=0)), C.byref(a), None) == -22


def test_table_coverage_check_matches_the_reference_rule():
    """The decode kernel's per-item guard `hist > 0 && (hist - 1) / bs >= cols` (an item
    that fails it reads no table entry and poisons its rows) is the reference's
    `ceil(prefix / bs) > cols` (streaming_attention.py:51-53) for every history length."""
    for bs in (32, 128, 1536):
        for cols in range(0, 6):
            for hist in range(0, 7 * bs + 2):
                assert (hist > 0 and (hist - 1) // bs >= cols) == (-(-hist // bs) > cols)


def prefill_args(**kw):
    """Continuation prefill arguments that pass every host check up to the table
    coverage (placeholder device addresses; nothing is launched)."""
    a = _lib.PrefillArgs(q=0x10000, q_stride_token=1536, k=0x20000, v=0x30000, kv_stride_token=256,
                         num_tokens=8, num_q_heads=6, num_kv_heads=1, head_dim=256, history=1000,
                         block_table_row=0x40000, scale=0.0625, out=0x50000, out_stride_token=1536,
                         workspace=0x100000, workspace_bytes=1 << 30, q_dtype=_lib.OSCAR_BF16)
    a.cache.k, a.cache.v = 0x100000, 0x200000
    a.cache.num_blocks, a.cache.block_size, a.cache.num_kv_heads, a.cache.head_dim = 8, 128, 1, 256
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_prefill_rejects_a_table_row_that_cannot_cover_the_history(lib):
    for history, cols in ((1000, 7), (129, 1), (1, 0)):
        a = prefill_args(history=history, block_table_cols=cols)
        assert lib.oscar_attn_prefill_v1(C.byref(a), None) == -22
        assert b"Block table cannot cover the history" in lib.oscar_last_error()


def step_args(qsl, seqs, has_new=True, rows=None, cols=16, staging_rows=None):
    """Native-step arguments with host metadata; device fields are placeholders.  The
    calls below are rejected by the host checks before the context or the stream is
    touched."""
    a = _lib.StepArgs(query=0x10000, num_tokens=qsl[-1], num_q_heads=6, q_dtype=_lib.OSCAR_BF16,
                      block_table=0x20000, block_table_stride=cols, rk=0x30000, rv=0x40000,
                      output=0x50000, workspace=0x60000, workspace_bytes=1 << 20)
    if has_new:
        a.key, a.value, a.kv_stride_token, a.slot_mapping = 0x70000, 0x80000, 256, 0x90000
    a.cache.k, a.cache.v = 0x100000, 0x200000
    a.cache.num_blocks, a.cache.block_size, a.cache.num_kv_heads, a.cache.head_dim = 64, 128, 1, 256
    keep = [(C.c_int32 * len(qsl))(*qsl), (C.c_int32 * len(seqs))(*seqs)]
    a.host_query_start_loc = C.cast(keep[0], C.c_void_p)
    a.host_seq_lens = C.cast(keep[1], C.c_void_p)
    a.num_reqs = len(seqs)
    a.block_table_rows = len(seqs) if rows is None else rows
    a.block_table_cols = cols
    if staging_rows is not None:
        st = _lib.Staging(stage_k=0xA0000, stage_v=0xB0000, owner=0xC0000, rows=staging_rows)
        keep.append(st)
        a.staging = C.pointer(st)
    return a, keep


def test_native_step_rejects_what_the_reference_rejects(lib):
    """oscar_decode_step_v1 raises where streaming_attention.py:48-65 raises: a missing
    table row, a history whose pages outnumber the table's columns (the history is
    seq minus the chunk with new K/V, seq without), an empty staging arena."""
    ctx = (C.c_uint8 * 4096)()  # never dereferenced: every call below fails its host checks
    cases = [
        (dict(qsl=[0, 4, 8], seqs=[1000, 1000], rows=1), b"Missing request block-table rows"),
        (dict(qsl=[0, 4, 8], seqs=[1000, 1000], cols=0), b"Missing request block-table rows"),
        # 2052 - 4 = 2048 history tokens fill exactly 16 pages; 2053 - 4 needs 17
        (dict(qsl=[0, 4, 8], seqs=[2052, 2053]), b"Block table cannot cover the history"),
        (dict(qsl=[0, 1, 2], seqs=[2048, 2049], has_new=False), b"Block table cannot cover the history"),
        (dict(qsl=[0, 4], seqs=[1000], staging_rows=0), b"Invalid streaming staging geometry"),
    ]
    for kw, msg in cases:
        a, keep = step_args(**kw)
        assert lib.oscar_decode_step_v1(C.cast(ctx, C.c_void_p), C.byref(a), None) == -22, kw
        assert msg in lib.oscar_last_error(), (kw, lib.oscar_last_error())
    # a request without queries in this batch reads nothing, whatever its length
    a, keep = step_args(qsl=[0, 4, 4], seqs=[1000, 99999], rows=2)
    a.block_table_rows = 1
    assert lib.oscar_decode_step_v1(C.cast(ctx, C.c_void_p), C.byref(a), None) == -22
    assert b"Missing request block-table rows" in lib.oscar_last_error()


def test_decode_rejects_a_workspace_smaller_than_the_plan_needs(lib):
    a = decode_args(workspace_bytes=4 * 32 * 257 * 4 - 16)
    assert lib.oscar_attn_decode_v1(C.byref(a), None) == -22
    assert b"workspace" in lib.oscar_last_error()
    a = decode_args(max_group_items=5)
    assert lib.oscar_attn_decode_v1(C.byref(a), None) == -22
    assert b"max_group_items" in lib.oscar_last_error()


def test_static_decode_rejects_plans_beyond_its_scratch(lib):
    a = decode_args(num_items=_lib.DECODE_STATIC_MAX_ITEMS + 1,
                    max_group_items=_lib.DECODE_STATIC_MAX_ITEMS + 1)
    assert lib.oscar_attn_decode_static_v1(C.byref(a), None) == -22
    assert b"static scratch" in lib.oscar_last_error()


# ---- the prefill's balanced split (oscar_prefill_plan_v1)
PREFILL_SPLIT_CASES = [
    (15360, 9256, 6, 1),   # config 5 continuation
    (0, 2048, 6, 1),       # config 5 fresh-only prefill
    (3000, 300, 6, 1), (129, 1024, 6, 1), (8193, 257, 6, 1),
    (0, 21, 6, 1),         # one query tile: nothing to split
    (0, 32768, 6, 1),      # long fresh prefill: the chunk count cap
    (500, 5000, 8, 2), (1, 70000, 1, 1), (40000, 5, 6, 1),
]


def prefill_plan(lib, history, n, hq, hk):
    out = (C.c_int32 * 64)()
    assert lib.oscar_prefill_plan_v1(history, n, hq, hk, out, 64) == 0
    chunks, U, ntq, qmin1, units, slots = list(out)[:6]
    return chunks, U, ntq, qmin1, units, slots, list(out)[6:6 + 33]


@pytest.mark.parametrize("history,n,hq,hk", PREFILL_SPLIT_CASES)
def test_prefill_split_covers_every_key_tile_once(lib, history, n, hq, hk):
    """The prefill kernel's unit decode (attn_prefill.hip: chunk class by base[], tile
    ntq - 1 - idx, key tiles [c U, min((c + 1) U, kt)), slot) over the plan: every query
    tile's key tiles [0, kt) are covered exactly once, the split tiles' partial slots are
    distinct and dense, the merge finds each chunk's slot by its own formula, and the
    workspace size is the history values plus one partial per slot."""
    group = hq // hk
    qtok = 128 // group
    chunks, U, ntq, qmin1, units, slots, base = prefill_plan(lib, history, n, hq, hk)
    assert ntq == -(-n // qtok) or chunks == 0
    kt = [-(-(history + min((qt + 1) * qtok, n)) // 32) for qt in range(-(-n // qtok))]
    hist_b = -(-2 * history * hk * 256 * 2 // 256) * 256 if history > 0 else 0
    ws = lib.oscar_prefill_workspace_bytes_v2(history, n, hq, hk, 256)
    if chunks < 2:
        assert chunks == 0 and ws == hist_b
        assert max(kt) <= max(16, -(-sum(kt) * hk // 512))  # the heaviest tile fits one chunk
        return
    assert U >= 16 and chunks == -(-kt[-1] // U) <= 32
    cover = {qt: [] for qt in range(ntq)}
    seen_slots = set()
    for u in range(units):
        c = max(cc for cc in range(chunks) if u >= base[cc])
        idx = u - base[c]
        qt = ntq - 1 - idx
        kb, ke = c * U, min(c * U + U, kt[qt])
        assert 0 <= qt < ntq and kb < ke
        slot = (idx if c == 0 else u - qmin1) if qt >= qmin1 else -1
        cover[qt].append((kb, ke, c, slot))
        if slot >= 0:
            assert slot not in seen_slots and 0 <= slot < slots
            seen_slots.add(slot)
            s = ntq - 1 - qt
            assert slot == (s if c == 0 else base[c] + s - qmin1)  # prefill_merge_kernel's slot
    assert len(seen_slots) == slots
    for qt, ranges in cover.items():
        ranges.sort()
        assert ranges[0][0] == 0 and ranges[-1][1] == kt[qt]
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
        split = len(ranges) > 1
        assert split == (qt >= qmin1) == (kt[qt] > U)
        assert all((r[3] >= 0) == split for r in ranges)
    # units are dealt chunk-major, heaviest tile first: unit sizes never grow within a class
    sizes = [min(U, kt[ntq - 1 - (u - base[c])] - c * U)
             for c in range(chunks) for u in range(base[c], base[c + 1])]
    assert sum(sizes) == sum(kt)
    assert ws == hist_b + slots * hk * 128 * 257 * 4
    assert ws >= (lib.oscar_prefill_workspace_bytes_v1(history, hk, 256) if history > 0 else 0)


def test_prefill_split_sizes_reject_bad_arguments(lib):
    out = (C.c_int32 * 64)()
    assert lib.oscar_prefill_plan_v1(0, 100, 6, 1, out, 10) == -22
    assert lib.oscar_prefill_plan_v1(0, 100, 5, 2, out, 64) == -22
    assert lib.oscar_prefill_workspace_bytes_v2(-1, 100, 6, 1, 256) == -22
    assert lib.oscar_prefill_workspace_bytes_v2(0, 100, 6, 1, 64) == -22
    assert lib.oscar_prefill_workspace_bytes_v2(0, 0, 6, 1, 256) == 0
