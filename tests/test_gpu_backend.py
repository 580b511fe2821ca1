"""The plugin impl's forward on the GPU against the oracle's restatement of the
reference backend (backend.py:249-393): writes, window tags, and attention routed to
fresh-only prefill, split-K decode / MTP and continuation prefill, in bf16 and fp16."""
import numpy as np
import pytest
import torch

from oracle import backend as ob
from oracle import cases

pytestmark = pytest.mark.gpu


class _Layer:
    layer_name = "model.layers.3.self_attn.attn"


class _MD:
    pass


@pytest.mark.parametrize("qdt,ulp", [(torch.bfloat16, 2.0 ** -7), (torch.float16, 2.0 ** -10)],
                         ids=["bf16", "fp16"])
def test_forward_steps_match_oracle(cuda, qdt, ulp):
    from oscar_amd.backend import OscarAttentionBackendImpl

    dev = torch.device("cuda", 0)
    d, hq, hk, bs = 256, 6, 1, 128
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_heads, impl.num_kv_heads, impl.scale = d, hq, hk, d ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    layer = _Layer()
    rk, rv = cases.hadamard_rotation(d, 5), cases.qr_rotation(d, 6)
    layer._oscar_rots = (torch.from_numpy(rk).to(dev), torch.from_numpy(rv).to(dev))
    nb, per = 24, 12
    caches = [torch.zeros(nb, bs, hk, d, dtype=torch.int8, device=dev) for _ in range(2)]
    table = np.random.default_rng(7).permutation(nb).reshape(2, per).astype(np.int32)
    oracle_layer = ob.OracleLayer(k8=np.zeros((nb, bs, hk, d), np.uint8), v8=np.zeros((nb, bs, hk, d), np.uint8),
                                  rk=rk, rv=rv, hq=hq, hk=hk, d=d, scale=d ** -0.5)
    q_dtype = "bf16" if qdt == torch.bfloat16 else "f16"
    lens = [0, 0]
    # (new tokens of request 0, of request 1): fresh prefills, MTP + single-token
    # decode, a continuation chunk (routed to the prefill) beside a decode
    for step, (n0, n1) in enumerate([(300, 700), (4, 1), (200, 1)]):
        news = [n0, n1]
        slots, qsl, seqs = [], [0], []
        for r, n in enumerate(news):
            pos = np.arange(lens[r], lens[r] + n)
            slots += (table[r, pos // bs].astype(np.int64) * bs + pos % bs).tolist()
            qsl.append(qsl[-1] + n)
            seqs.append(lens[r] + n)
        N = qsl[-1]
        q = cases.bf16_normal((N, hq, d), 100 + step)
        k = cases.kv_outliers(N, hk, d, 200 + step)
        v = cases.kv_outliers(N, hk, d, 300 + step)
        md = _MD()
        md.num_actual_tokens = N
        md.slot_mapping = torch.tensor(slots, device=dev)
        md.query_start_loc_cpu = torch.tensor(qsl)
        md.seq_lens_list = seqs
        md.block_tables = torch.from_numpy(table).to(dev)
        out = torch.empty(N, hq * d, dtype=qdt, device=dev)
        tq, tk, tv = (torch.from_numpy(x).to(dev).to(qdt) for x in (q, k, v))
        impl.forward(layer, tq.view(N, -1), tk.view(N, -1), tv.view(N, -1), caches, md, output=out)
        torch.cuda.synchronize()
        ref = ob.forward(oracle_layer, q, k, v, slots, qsl, seqs, table, q_dtype=q_dtype)
        got = out.float().view(N, hq, d).cpu().numpy()
        # 2e-2 absolute plus one output ulp of the value (outlier channels make early
        # causal rows large, where one ulp exceeds 2e-2)
        excess = float((np.abs(got - ref) - (2e-2 + ulp * np.abs(ref))).max())
        print(f"{q_dtype} step {step}: max|out - oracle| = {np.abs(got - ref).max():.3e}", flush=True)
        assert excess <= 0, f"step {step}: output differs from the oracle"
        lens = seqs
    assert np.array_equal(layer._oscar_slot_owner.cpu().numpy(), oracle_layer.staging.owner)
    assert np.array_equal(caches[0].view(torch.uint8).cpu().numpy(), oracle_layer.k8)
    assert np.array_equal(caches[1].view(torch.uint8).cpu().numpy(), oracle_layer.v8)
