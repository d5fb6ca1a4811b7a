"""GPU: torch.compile(backend=get_npu_backend(mode="reduce-overhead")) lowers onto the HIP ops and
captures a hipGraph; replays with new device values (activations, sequence lengths, block tables,
group lists, cache slots) are checked against eager and the oracle on every replay, with eager
work and synchronisations in between. This is the role of the reference's graph_task_update
(python/torchair/_acl_concrete_graph/acl_graph.py:542-577): data-dependent sizes are read on the
device, so a replay with new values needs no re-capture."""
import math

import numpy as np
import pytest
import torch

import torchair_amd
from oracle import golden as G
from tests.helpers import assert_close, f32np
from torchair_amd import graph as tai_graph

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _backend():
    cfg = torchair_amd.CompilerConfig()
    cfg.mode = "reduce-overhead"
    return torchair_amd.get_npu_backend(compiler_config=cfg)


def _churn():
    """Unrelated eager work and a host synchronisation between replays."""
    a = torch.randn(1 << 20, device=DEV)
    (a * 3).sum().item()
    torch.cuda.synchronize()


class _Mlp(torch.nn.Module):
    """Config-1 W8A8 SwiGLU MLP; the weights are parameters, so the graph uses them in place."""

    def __init__(self, h, inter, g):
        super().__init__()
        p = lambda t: torch.nn.Parameter(t.to(DEV), requires_grad=False)  # noqa: E731
        self.wgu = p(torch.randint(-127, 128, (h, 2 * inter), generator=g, dtype=torch.int8))
        self.sgu = p(torch.rand(2 * inter, generator=g) * 9e-3 + 1e-3)
        self.wd = p(torch.randint(-127, 128, (inter, h), generator=g, dtype=torch.int8))
        self.sd = p(torch.rand(h, generator=g) * 9e-3 + 1e-3)
        self.one = p(torch.ones(1))

    def forward(self, x):
        npu = torch.ops.npu
        q, s = npu.npu_dynamic_quant(x)
        h = npu.npu_quant_matmul(q, self.wgu, self.one, output_dtype=torch.int32)
        q2, s2 = npu.npu_dequant_swiglu_quant(h, weight_scale=self.sgu, activation_scale=s, quant_mode=1,
                                              activate_left=True)
        return npu.npu_quant_matmul(q2, self.wd, self.sd, pertoken_scale=s2, output_dtype=torch.bfloat16)


def test_compiled_mlp_cfg1_captures_and_replays():
    g = torch.Generator().manual_seed(50)
    t, h, inter = 128, 2048, 5632
    mod = _Mlp(h, inter, g)
    fn = torch.compile(mod, backend=_backend(), fullgraph=True)
    caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
    for i in range(4):
        x = torch.randn(t, h, generator=g).to(torch.bfloat16)
        got = fn(x.to(DEV)).clone()
        want = mod(x.to(DEV))
        assert torch.equal(got, want), f"call {i}: graph differs from eager"
        if i in (0, 3):  # the oracle on the first and the last replay
            wq, ws = G.dynamic_quant(f32np(x))
            acc = G.quant_matmul(wq, mod.wgu.cpu().numpy(), out_dtype="int32")
            q2, s2 = G.dequant_swiglu_quant(acc, mod.sgu.cpu().numpy(), ws, activate_left=True)
            ref = G.quant_matmul(q2, mod.wd.cpu().numpy(), mod.sd.cpu().numpy(), s2, None, "bf16")
            assert_close(f32np(got), ref, rtol=2e-2, atol=2e-2)
        _churn()
    assert tai_graph.stats["captures"] == caps + 1
    assert tai_graph.stats["eager_fallbacks"] == falls


def _paged(g, lens, nb_total, width, bs, hkv, d):
    perm = torch.randperm(nb_total, generator=g).to(torch.int32)
    bt = torch.zeros(len(lens), width, dtype=torch.int32)
    off = 0
    for b, L in enumerate(lens):
        n = (L + bs - 1) // bs
        bt[b, :n] = perm[off:off + n]
        off += n
    return bt


def test_compiled_decode_replays_with_new_lengths_and_block_table():
    g = torch.Generator().manual_seed(51)
    b, hq, hkv, d, bs, width = 8, 32, 8, 128, 128, 16
    nblk = b * width
    kc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16)
    vc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16)
    kcd, vcd = kc.to(DEV), vc.to(DEV)

    def step(q, lens, bt):
        return torch.ops.air.npu_fused_infer_attention_score(
            q, kcd, vcd, actual_seq_lengths_kv=lens, block_table=bt, num_heads=hq, num_key_value_heads=hkv,
            input_layout="BSH", block_size=bs, scale=1.0 / math.sqrt(d))[0]

    fn = torch.compile(step, backend=_backend(), fullgraph=True)
    caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
    for i in range(4):
        lens = torch.randint(1, width * bs + 1, (b,), generator=g)
        if i == 2:
            lens[3] = 0  # an empty sequence
        bt = _paged(g, lens.tolist(), nblk, width, bs, hkv, d)
        q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16)
        got = fn(q.to(DEV), lens.to(DEV), bt.to(DEV)).clone()
        want = step(q.to(DEV), lens.to(DEV), bt.to(DEV))
        assert torch.equal(got, want), f"replay {i} differs from eager"
        ref, _ = G.paged_decode_attention(f32np(q).reshape(b, hq, d), f32np(kc).reshape(nblk, bs, hkv, d),
                                          f32np(vc).reshape(nblk, bs, hkv, d), bt.numpy(), lens.numpy(),
                                          1.0 / math.sqrt(d))
        assert_close(f32np(got).reshape(b, hq, d), ref)
        _churn()
    assert tai_graph.stats["captures"] == caps + 1
    assert tai_graph.stats["eager_fallbacks"] == falls


def test_compiled_fia_with_list_lengths_is_captured():
    """npu:: FIA with int-list lengths: the lengths are constants of the captured graph."""
    g = torch.Generator().manual_seed(52)
    b, hq, hkv, d, bs, width = 4, 8, 2, 128, 64, 8
    lens = [100, 1, 512, 300]
    nblk = b * width
    kc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    bt = _paged(g, lens, nblk, width, bs, hkv, d).to(DEV)

    def step(q):
        return torch.ops.npu.npu_fused_infer_attention_score(
            q, kc, vc, actual_seq_lengths_kv=lens, block_table=bt, num_heads=hq, num_key_value_heads=hkv,
            input_layout="BSH", block_size=bs, scale=1.0 / math.sqrt(d))[0]

    fn = torch.compile(step, backend=_backend(), fullgraph=True)
    caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
    for i in range(3):
        q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16).to(DEV)
        got = fn(q).clone()
        assert torch.equal(got, step(q)), f"replay {i}"
        _churn()
    assert tai_graph.stats["captures"] == caps + 1
    assert tai_graph.stats["eager_fallbacks"] == falls


def test_compiled_grouped_matmul_replays_with_new_group_list():
    g = torch.Generator().manual_seed(53)
    e, k, n, m = 16, 512, 768, 2000
    w = torch.nn.Parameter(torch.randint(-127, 128, (e, k, n), generator=g, dtype=torch.int8).to(DEV),
                           requires_grad=False)

    def step(x, gl):
        return torch.ops.npu.npu_grouped_matmul([x], [w], group_list=gl, split_item=3, group_type=0,
                                                group_list_type=1, output_dtype=torch.int32)[0]

    fn = torch.compile(step, backend=_backend(), fullgraph=True)
    caps = tai_graph.stats["captures"]
    for i in range(4):
        x = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
        hi = e if i % 2 else e // 4  # alternately all experts live, then a quarter of them with long groups
        counts = torch.bincount(torch.randint(0, hi, (m - 50,), generator=g), minlength=e).to(torch.int64)
        got = fn(x.to(DEV), counts.to(DEV)).clone()
        want = G.grouped_matmul(x.numpy(), w.cpu().numpy(), counts.numpy(), 1, out_dtype="int32")
        rows = int(counts.sum())
        np.testing.assert_array_equal(got.cpu().numpy()[:rows], want[:rows], err_msg=f"replay {i}")
        _churn()
    assert tai_graph.stats["captures"] == caps + 1


def test_compiled_cache_write_updates_the_callers_cache():
    """A compiled decode step that scatters into the KV cache: the cache is written in place (not a
    clone), on the capture call and on every replay, exactly as eager writes it."""
    g = torch.Generator().manual_seed(54)
    t, hkv, d, nblk, bs = 16, 8, 128, 64, 32
    kc = torch.zeros(nblk, bs, hkv, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    kc_ref, vc_ref = kc.clone(), vc.clone()

    def step(key, value, kcache, vcache, slots):
        torch.ops.npu.npu_scatter_pa_kv_cache(key, value, kcache, vcache, slots)
        return key.float().sum()

    fn = torch.compile(step, backend=_backend(), fullgraph=True)
    caps = tai_graph.stats["captures"]
    perm = torch.randperm(nblk * bs, generator=g)
    for i in range(4):
        key = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
        val = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
        slots = perm[i * t:(i + 1) * t].to(DEV)
        fn(key, val, kc, vc, slots)
        step(key, val, kc_ref, vc_ref, slots)
        torch.cuda.synchronize()
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"call {i}: cache differs from eager"
        s = slots.cpu()
        assert torch.equal(kc.view(-1, hkv, d)[s.to(DEV)], key)
        _churn()
    assert tai_graph.stats["captures"] == caps + 1
    # a cache at another address is captured anew (it is part of the graph by pointer)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    key = torch.randn(t, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    fn(key, key, kc2, vc2, perm[:t].to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(kc2.view(-1, hkv, d)[perm[:t].to(DEV)], key)
    assert tai_graph.stats["captures"] == caps + 2


class _MoeFront(torch.nn.Module):
    """Gating, routing, per-token quant and the gate_up grouped GEMM of a MoE layer; the pattern pass
    folds the quant into the routing op (quant_mode 1)."""

    def __init__(self, h, e, inter, g):
        super().__init__()
        p = lambda t: torch.nn.Parameter(t.to(DEV), requires_grad=False)  # noqa: E731
        self.bias = p(torch.randn(e, generator=g) * 0.1)
        self.w = p(torch.randint(-127, 128, (e, h, 2 * inter), generator=g, dtype=torch.int8))
        self.e = e

    def forward(self, x, logits):
        npu = torch.ops.npu
        _, idx, _ = npu.npu_moe_gating_top_k(logits, 8, bias=self.bias, k_group=4, group_count=8, group_select_mode=1,
                                             renorm=0, norm_type=1, routed_scaling_factor=1.0, eps=1e-20)
        ex, ri, counts, _ = npu.npu_moe_init_routing_v2(x, idx, active_num=x.shape[0] * 8, expert_num=self.e,
                                                        expert_tokens_num_type=1, expert_tokens_num_flag=True,
                                                        row_idx_type=0)
        q, s = npu.npu_dynamic_quant(ex)
        acc = npu.npu_grouped_matmul([q], [self.w], group_list=counts, split_item=3, group_type=0, group_list_type=1,
                                     output_dtype=torch.int32)[0]
        return acc, s, ri, counts


def test_compiled_moe_front_folds_the_quant_into_routing():
    from torchair_amd import patterns
    g = torch.Generator().manual_seed(51)
    t, h, e, inter = 512, 1024, 64, 256
    mod = _MoeFront(h, e, inter, g)
    fused0 = patterns.stats["init_routing_dynamic_quant"]
    fn = torch.compile(mod, backend=_backend(), fullgraph=True)
    caps = tai_graph.stats["captures"]
    for i in range(3):
        x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(DEV)
        logits = torch.randn(t, e, generator=g).to(DEV)
        got = [o.clone() for o in fn(x, logits)]
        want = mod(x, logits)
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"call {i}: compiled front differs from eager"
        _churn()
    assert patterns.stats["init_routing_dynamic_quant"] == fused0 + 1
    assert tai_graph.stats["captures"] == caps + 1


class _Quant(torch.nn.Module):
    def forward(self, x):
        return torch.ops.npu.npu_dynamic_quant(x)


def test_compiled_inputs_by_address_replay_in_place_and_copy_a_moved_input():
    """debug.aclgraph.clone_input = False: the graph reads the caller's input tensor itself. New values
    written into the same tensor replay without a copy or a capture. A fresh tensor at another address
    (neither a parameter nor written in place) is copied into the capture-time tensor and replayed, as
    the reference does with its retained user inputs (acl_graph.py:1319-1337): the capture count stays
    at one over a loop of fresh inputs."""
    cfg = torchair_amd.CompilerConfig()
    cfg.mode = "reduce-overhead"
    cfg.debug.aclgraph.clone_input = False
    fn = torch.compile(_Quant(), backend=torchair_amd.get_npu_backend(compiler_config=cfg), fullgraph=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(70)
    xa = torch.randn(64, 512, generator=g, device=DEV).to(torch.bfloat16)

    def check(x):
        want_q, want_s = torch.ops.npu.npu_dynamic_quant(x.clone())
        q, s = fn(x)
        assert torch.equal(q, want_q) and torch.equal(s, want_s)

    c0 = tai_graph.stats["captures"]
    check(xa)
    c1 = tai_graph.stats["captures"]
    assert c1 == c0 + 1
    for _ in range(2):
        xa.copy_(torch.randn(64, 512, generator=g, device=DEV).to(torch.bfloat16))
        _churn()
        check(xa)
    for _ in range(4):
        xb = torch.randn(64, 512, generator=g, device=DEV).to(torch.bfloat16)
        _churn()
        check(xb)
    assert tai_graph.stats["captures"] == c1


def test_compiled_packed_tnd_chunked_prefill_is_captured():
    """Packed TND queries over a paged cache with host-list cumulative ends (constants of the captured
    graph) and an int8 attention_out: each replay equals eager."""
    g = torch.Generator().manual_seed(53)
    hq, hkv, d, bs, width = 8, 2, 128, 64, 8
    lk = [100, 1, 300, 64]
    lq = [2, 1, 5, 3]
    b = len(lk)
    cq = np.cumsum(lq).tolist()
    nblk = b * width
    kc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    bt = _paged(g, lk, nblk, width, bs, hkv, d).to(DEV)
    qs = torch.tensor([25.0], device=DEV)

    def step(q):
        return torch.ops.npu.npu_fused_infer_attention_score(
            q, kc, vc, actual_seq_lengths=cq, actual_seq_lengths_kv=lk, block_table=bt, num_heads=hq,
            num_key_value_heads=hkv, input_layout="TND", block_size=bs, scale=1.0 / math.sqrt(d), sparse_mode=3,
            quant_scale2=qs)[0]

    fn = torch.compile(step, backend=_backend(), fullgraph=True)
    caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
    for i in range(3):
        q = torch.randn(sum(lq), hq, d, generator=g).to(torch.bfloat16).to(DEV)
        got = fn(q).clone()
        assert got.dtype == torch.int8
        assert torch.equal(got, step(q)), f"replay {i}"
        _churn()
    assert tai_graph.stats["captures"] == caps + 1
    assert tai_graph.stats["eager_fallbacks"] == falls


def test_compiled_int8_query_and_learnable_sink_are_captured():
    """The int8 query (UINT64 dequant scales, converted inside the op) and the v2 learnable_sink, each
    captured once and equal to eager on every replay."""
    g = torch.Generator().manual_seed(54)
    b, s, hq, hkv, d = 2, 16, 4, 2, 64
    k8 = torch.randint(-128, 128, (b, s, hkv * d), generator=g, dtype=torch.int8).to(DEV)
    v8 = torch.randint(-128, 128, (b, s, hkv * d), generator=g, dtype=torch.int8).to(DEV)

    def u64(x):
        return torch.tensor([int(np.array([x], np.float32).view(np.uint32)[0])], dtype=torch.int64, device=DEV)

    d1, q1, d2 = u64(4e-4), torch.tensor([127.0], device=DEV), u64(1e-4)

    def step_q8(q):
        return torch.ops.air.npu_fused_infer_attention_score(
            q, k8, v8, num_heads=hq, num_key_value_heads=hkv, input_layout="BSH", scale=1 / math.sqrt(d),
            sparse_mode=3, dequant_scale1=d1, quant_scale1=q1, dequant_scale2=d2)[0]

    kb = torch.randn(b, s, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    vb = torch.randn(b, s, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    sink = torch.randn(hq, generator=g).to(torch.bfloat16).to(DEV)

    def step_sink(q):
        return torch.ops.air.npu_fused_infer_attention_score_v2(
            q, kb, vb, num_query_heads=hq, num_key_value_heads=hkv, input_layout="BSH",
            softmax_scale=1 / math.sqrt(d), sparse_mode=3, learnable_sink=sink)[0]

    for step, make in ((step_q8, lambda: torch.randint(-128, 128, (b, s, hq * d), generator=g, dtype=torch.int8)),
                       (step_sink, lambda: torch.randn(b, s, hq * d, generator=g).to(torch.bfloat16))):
        fn = torch.compile(step, backend=_backend(), fullgraph=True)
        caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
        for i in range(3):
            q = make().to(DEV)
            got = fn(q).clone()
            assert torch.equal(got, step(q)), f"{step.__name__} replay {i}"
            _churn()
        assert tai_graph.stats["captures"] == caps + 1
        assert tai_graph.stats["eager_fallbacks"] == falls


def test_compiled_int8_cache_and_sink_decode_replay_with_new_lengths():
    """The one-token decode over int8 caches (pages widened in the workspace, then the decode kernel) and
    with a learnable_sink (taken in by the merge) captured once each; every replay, with new lengths and
    block tables, equals the eager call."""
    g = torch.Generator().manual_seed(53)
    b, hq, hkv, d, bs, width = 8, 32, 8, 128, 64, 16
    nblk = b * width
    k8 = torch.randint(-128, 128, (nblk, bs, hkv * d), generator=g, dtype=torch.int8).to(DEV)
    v8 = torch.randint(-128, 128, (nblk, bs, hkv * d), generator=g, dtype=torch.int8).to(DEV)
    ks = (torch.rand(hkv * d, generator=g) * 0.02 + 0.005).to(DEV)
    vs = (torch.rand(hkv * d, generator=g) * 0.02 + 0.005).to(DEV)
    kc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(nblk, bs, hkv * d, generator=g).to(torch.bfloat16).to(DEV)
    sink = (torch.randn(hq, generator=g) * 2).to(torch.bfloat16).to(DEV)

    def step8(q, lens, bt):
        return torch.ops.air.npu_fused_infer_attention_score(
            q, k8, v8, actual_seq_lengths_kv=lens, block_table=bt, num_heads=hq, num_key_value_heads=hkv,
            input_layout="BSH", block_size=bs, scale=1.0 / math.sqrt(d), key_antiquant_scale=ks,
            value_antiquant_scale=vs)[0]

    def step_sink(q, lens, bt):
        return torch.ops.air.npu_fused_infer_attention_score_v2(
            q, kc, vc, actual_seq_kvlen=lens, block_table=bt, num_query_heads=hq, num_key_value_heads=hkv,
            input_layout="BSH", block_size=bs, softmax_scale=1.0 / math.sqrt(d), learnable_sink=sink)[0]

    for step in (step8, step_sink):
        fn = torch.compile(step, backend=_backend(), fullgraph=True)
        caps, falls = tai_graph.stats["captures"], tai_graph.stats["eager_fallbacks"]
        for i in range(4):
            lens = torch.randint(1, width * bs + 1, (b,), generator=g)
            if i == 2:
                lens[3] = 0  # an empty sequence
            bt = _paged(g, lens.tolist(), nblk, width, bs, hkv, d)
            q = torch.randn(b, 1, hq * d, generator=g).to(torch.bfloat16)
            print("case", step.__name__, "replay", i, flush=True)
            got = fn(q.to(DEV), lens.to(DEV), bt.to(DEV)).clone()
            want = step(q.to(DEV), lens.to(DEV), bt.to(DEV))
            assert torch.equal(got, want), f"{step.__name__}: replay {i} differs from eager"
            _churn()
        assert tai_graph.stats["captures"] == caps + 1
        assert tai_graph.stats["eager_fallbacks"] == falls
