"""torch.ops.oscar_amd registration: schemas, mutated arguments and the fake (meta)
implementations on the CPU; the GPU tests call the operators against the direct
wrappers (same kernels, same bits) and run torch.library.opcheck."""
import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import oscar_amd.torch_ops  # noqa: F401  (registers the operators)
from oracle import cases

OPS = ("rotate", "store", "attention_decode", "attention_prefill")


def test_operators_are_registered_with_their_schemas():
    for name in OPS:
        schema = str(getattr(torch.ops.oscar_amd, name).default._schema)
        assert schema.startswith(f"oscar_amd::{name}(")
    import re

    store = str(torch.ops.oscar_amd.store.default._schema)
    mutated = set(re.findall(r"Tensor\(a\d+!\)\?? (\w+)", store))
    assert mutated == {"k_cache", "v_cache", "stage_k", "stage_v", "owner"}, store
    assert store.endswith("-> ()")


def test_fake_kernels_give_the_output_shapes():
    with FakeTensorMode():
        q = torch.empty(4, 6, 256, dtype=torch.bfloat16, device="cuda")
        kc = torch.empty(8, 128, 1, 256, dtype=torch.int8, device="cuda")
        bt = torch.empty(1, 8, dtype=torch.int32, device="cuda")
        o, lse = torch.ops.oscar_amd.attention_decode(q, None, None, kc, kc, bt, [0, 4], [100], 0.0625, 256)
        assert o.shape == (4, 6, 256) and o.dtype == torch.float32 and lse.shape == (4, 6)
        r = torch.ops.oscar_amd.rotate(q, torch.empty(256, 256, device="cuda"), True)
        assert r.shape == q.shape and r.dtype == q.dtype
        out, lse = torch.ops.oscar_amd.attention_prefill(q, q[:, :1], q[:, :1], 0.0625, 256, 100, kc, kc, bt[0])
        assert out.dtype == torch.float32 and lse.shape == (4, 6)
        out, lse = torch.ops.oscar_amd.attention_prefill(q, q[:, :1], q[:, :1], 0.0625, 256)
        assert out.dtype == torch.bfloat16 and out.shape == (4, 6, 256) and lse.numel() == 0


@pytest.mark.gpu
def test_operators_match_the_direct_wrappers():
    from oscar_amd import ops

    d, hq, hk, bs, nb, n = 256, 6, 1, 128, 8, 48
    g = torch.Generator(device="cuda").manual_seed(5)
    r = torch.from_numpy(cases.hadamard_rotation(d, 3)).cuda()
    x = torch.randn(n, hq, d, generator=g, device="cuda").bfloat16()
    assert torch.equal(torch.ops.oscar_amd.rotate(x, r, False), ops.rotate(x, r))
    torch.library.opcheck(torch.ops.oscar_amd.rotate, (x, r, True))
    # store through the operator and through the wrapper: identical caches
    k = torch.randn(n, hk, d, generator=g, device="cuda").bfloat16()
    v = torch.randn(n, hk, d, generator=g, device="cuda").bfloat16()
    slots = torch.randperm(nb * bs, device="cuda")[:n].to(torch.int64)
    caches = [torch.zeros(nb, bs, hk, d, dtype=torch.int8, device="cuda") for _ in range(4)]
    torch.ops.oscar_amd.store(k, v, caches[0], caches[1], slots, None, None, None, d, r, r)
    ops.store(k, v, caches[2], caches[3], slots, head_dim=d, rk=r, rv=r)
    torch.cuda.synchronize()
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3]) and caches[0].any()
    # decode over that history (one request, 4 new queries; no current chunk)
    seq = n  # positions 0..n-1 of one request over every block (slots are random, values too)
    q = torch.randn(4, hq, d, generator=g, device="cuda").bfloat16()
    bt = torch.arange(nb, dtype=torch.int32, device="cuda")[None]
    o1, l1 = torch.ops.oscar_amd.attention_decode(q, None, None, caches[0], caches[1], bt, [0, 4], [seq], 0.0625, d)
    plan = ops.plan_decode([0, 4], [seq], has_new=False, num_kv_heads=hk, group=hq // hk, head_dim=d,
                           device=q.device)
    o2, l2 = ops.attention_decode(q, None, None, caches[0], caches[1], bt, plan, 0.0625, head_dim=d)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2) and torch.isfinite(o1).all()
