"""CPU checks of the drop-in boundary: the C ABI library, op schemas and meta rules, the
converter extension surface and the Dynamo backend on the CPU debug path."""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import torchair_amd
from torchair_amd import CompilerConfig, _lib, get_npu_backend, register_fx_node_ge_converter
from torchair_amd.converter import _get_converter
from torchair_amd.npu_fx_compiler import lower_graph

ROOT = Path(__file__).resolve().parent.parent


def _header_symbols():
    text = (ROOT / "include" / "tai_kernels.h").read_text()
    return sorted(set(re.findall(r"\b(tai_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    syms = _header_symbols()
    assert len(syms) >= 17
    for s in syms:
        assert hasattr(lib, s), f"{s} missing from libtai_kernels.so"
    assert set(syms) == set(_lib.exported_symbols())
    assert lib.tai_abi_version() == 1
    # the ctypes mirror of the attention argument struct has the library's size
    assert lib.tai_fia_general_args_size() == __import__("ctypes").sizeof(_lib.FiaGeneralArgs)


def test_library_build_id_matches_sources_and_stale_library_is_refused():
    from torchair_amd import _build
    lib = _lib.load()
    assert lib.tai_build_id().decode() == _build.source_id()

    class _Stale:
        @staticmethod
        def tai_build_id():
            return b"0000"
    with pytest.raises(RuntimeError, match="stale"):
        _lib._check_fresh(_Stale())


def test_library_rejects_bad_arguments_without_gpu():
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.call("tai_dynamic_quant", 1, 99, 4, 4, None, None, -1, 0, 1, 1, None)
    with pytest.raises(RuntimeError, match="last dim must be even"):
        _lib.call("tai_dequant_swiglu_quant", 1, 4, 7, None, None, None, -1, None, None, -1, 0, 0, 1, 1, None)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("tai_grouped_matmul", 1, 1, 4, 16, 16, 2, 0, 1, 0, None, None, None, -1, 3, 1, None, 0, None)
    with pytest.raises(RuntimeError, match="drop-pad"):
        _lib.call("tai_moe_finalize_routing", 1, 15, 4, 8, 2, None, None, None, None, -1, 1, None, 1, 1, None)
    assert _lib.query("tai_grouped_matmul_workspace_size", 32768, 4096, 256) > 0


def test_ops_refuse_cpu_tensors_without_the_debug_path():
    x = torch.randn(4, 16)
    if torch.ops.npu.npu_dynamic_quant.default.has_kernel_for_dispatch_key("CPU"):
        pytest.skip("oracle CPU kernels registered in this process")
    with pytest.raises(NotImplementedError):
        torch.ops.npu.npu_dynamic_quant(x)


def test_meta_shapes_follow_reference_rules():
    m = torch.device("meta")
    y, s = torch.ops.npu.npu_dynamic_quant(torch.empty(3, 5, 64, device=m, dtype=torch.bfloat16))
    assert y.shape == (3, 5, 64) and y.dtype == torch.int8 and s.shape == (3, 5)
    y, s = torch.ops.npu.npu_dequant_swiglu_quant(torch.empty(128, 11264, device=m, dtype=torch.int32), quant_mode=1)
    assert y.shape == (128, 5632) and s.shape == (128,)
    with pytest.raises(RuntimeError, match="even"):
        torch.ops.npu.npu_dequant_swiglu_quant(torch.empty(4, 7, device=m, dtype=torch.int32))
    out = torch.ops.npu.npu_quant_matmul(torch.empty(128, 2048, device=m, dtype=torch.int8),
                                         torch.empty(2048, 11264, device=m, dtype=torch.int8),
                                         torch.empty(1, device=m), output_dtype=torch.int32)
    assert out.shape == (128, 11264) and out.dtype == torch.int32
    y, idx, o = torch.ops.npu.npu_moe_gating_top_k(torch.empty(4096, 256, device=m), 8)
    assert y.shape == (4096, 8) and idx.dtype == torch.int32 and o.shape == (4096, 256)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(torch.empty(4096, 7168, device=m, dtype=torch.bfloat16),
                                                            torch.empty(4096, 8, device=m, dtype=torch.int32),
                                                            expert_num=256)
    assert ex.shape == (32768, 7168) and ri.shape == (32768,) and tok.shape == (256,)
    ex, ri, tok, es = torch.ops.npu.npu_moe_init_routing_v2(torch.empty(4096, 7168, device=m, dtype=torch.bfloat16),
                                                            torch.empty(4096, 8, device=m, dtype=torch.int32),
                                                            expert_num=256, quant_mode=1)
    assert ex.dtype == torch.int8 and es.shape == (32768,) and es.dtype == torch.float32
    q = torch.empty(64, 1, 32 * 128, device=m, dtype=torch.bfloat16)
    kc = torch.empty(100, 128, 8 * 128, device=m, dtype=torch.bfloat16)
    out, lse = torch.ops.air.npu_fused_infer_attention_score(
        q, kc, kc, block_table=torch.empty(64, 32, device=m, dtype=torch.int32), num_heads=32,
        num_key_value_heads=8, input_layout="BSH", block_size=128, softmax_lse_flag=True)
    assert out.shape == (64, 1, 4096) and lse.shape == (64, 32, 1, 1)
    qn = torch.empty(128, 1, 128, 512, device=m, dtype=torch.bfloat16)
    lat = torch.empty(10, 128, 1, 512, device=m, dtype=torch.int8)
    out, lse = torch.ops.npu.npu_fused_infer_attention_score(
        qn, lat, lat, block_table=torch.empty(128, 64, device=m, dtype=torch.int32), num_heads=128,
        num_key_value_heads=1, input_layout="BSND", query_rope=torch.empty(128, 1, 128, 64, device=m,
                                                                            dtype=torch.bfloat16))
    assert out.shape == (128, 1, 128, 512) and out.dtype == torch.bfloat16 and lse.shape == (0,)


def test_converter_registration_surface():
    conv = _get_converter(torch.ops.npu.npu_dynamic_quant.default)
    assert conv is not None and conv.require_meta is True

    lib = torch.library.Library("tai_test", "FRAGMENT")
    lib.define("twice(Tensor x) -> Tensor")
    lib.impl("twice", lambda x: x * 2, "CompositeExplicitAutograd")

    @register_fx_node_ge_converter(torch.ops.tai_test.twice.default)
    def convert_twice(x, meta_outputs=None):
        assert meta_outputs is not None and meta_outputs.shape == x.node.meta["val"].shape
        return torch.ops.aten.add.Tensor(x, x)

    assert _get_converter(torch.ops.tai_test.twice.default).require_meta is True
    assert register_fx_node_ge_converter(None)(lambda: 1) is None


def test_backend_lowers_user_converter_and_runs_on_cpu():
    lib = torch.library.Library("tai_test2", "FRAGMENT")
    lib.define("scaled(Tensor x, float s) -> Tensor")
    lib.impl("scaled", lambda x, s: x * 1000.0, "CompositeExplicitAutograd")  # deliberately wrong eager impl

    @register_fx_node_ge_converter(torch.ops.tai_test2.scaled.default)
    def convert_scaled(x, s, meta_outputs=None):
        return torch.ops.aten.mul.Tensor(x, s)

    def f(x):
        return torch.ops.tai_test2.scaled(x, 3.0) + 1

    cfg = CompilerConfig()
    cfg.mode = "reduce-overhead"
    fn = torch.compile(f, backend=get_npu_backend(compiler_config=cfg), fullgraph=True)
    x = torch.randn(5)
    torch.testing.assert_close(fn(x), x * 3 + 1)  # the converter, not the eager impl, ran


def test_cpu_debug_path_mlp_matches_oracle():
    """cfg1 composition through torch.compile(backend=get_npu_backend()) on CPU (oracle kernels)."""
    from oracle import cpu_ops, golden as G
    cpu_ops.register()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 64, generator=g).to(torch.bfloat16)
    wgu = torch.randint(-127, 128, (64, 96), generator=g, dtype=torch.int8)
    sgu = torch.rand(96, generator=g) * 9e-3 + 1e-3
    wd = torch.randint(-127, 128, (48, 64), generator=g, dtype=torch.int8)
    sd = torch.rand(64, generator=g) * 9e-3 + 1e-3

    def mlp(x):
        q, s = torch.ops.npu.npu_dynamic_quant(x)
        h = torch.ops.npu.npu_quant_matmul(q, wgu, torch.ones(1), output_dtype=torch.int32)
        q2, s2 = torch.ops.npu.npu_dequant_swiglu_quant(h, weight_scale=sgu, activation_scale=s, quant_mode=1,
                                                        activate_left=True)
        return torch.ops.npu.npu_quant_matmul(q2, wd, sd, pertoken_scale=s2, output_dtype=torch.bfloat16)

    fn = torch.compile(mlp, backend=get_npu_backend(), fullgraph=True)
    got = fn(x)
    q, s = G.dynamic_quant(x.float().numpy())
    h = G.quant_matmul(q, wgu.numpy(), out_dtype="int32")
    q2, s2 = G.dequant_swiglu_quant(h, sgu.numpy(), s, activate_left=True)
    want = G.quant_matmul(q2, wd.numpy(), sd.numpy(), s2, None, "bf16")
    np.testing.assert_array_equal(got.float().numpy(), want)


def test_lowering_keeps_fused_nodes():
    gm = torch.fx.symbolic_trace(lambda x: torch.ops.npu.npu_dynamic_quant(x)[0])
    low = lower_graph(gm)
    targets = [n.target for n in low.graph.nodes if n.op == "call_function"]
    assert torch.ops.npu.npu_dynamic_quant.default in targets or torch.ops.npu.npu_dynamic_quant in targets


def test_compiler_config_validation():
    cfg = CompilerConfig()
    assert cfg.mode.value == "max-autotune"
    cfg.mode = "npugraph_ex"
    with pytest.raises(ValueError):
        cfg.mode = "fast"
    cfg.debug.aclgraph.static_capture_size_limit = 4
    with pytest.raises(ValueError):
        cfg.debug.aclgraph.static_capture_size_limit = 0
    assert CompilerConfig() != cfg and CompilerConfig() == CompilerConfig()
    assert torchair_amd.get_compiler(cfg).config is cfg


def test_pattern_pass_fuses_add_rms_norm_dynamic_quant_on_cpu():
    """add_rms_norm + dynamic_quant becomes the fused op (python/torchair/patterns/add_rms_norm_dynamic_quant.py)
    and the compiled result equals the eager composition, bit for bit."""
    from oracle import cpu_ops
    from torchair_amd.patterns import fuse_add_rms_norm_dynamic_quant
    cpu_ops.register()
    g = torch.Generator().manual_seed(3)
    x1, x2 = torch.randn(8, 64, generator=g).to(torch.bfloat16), torch.randn(8, 64, generator=g).to(torch.bfloat16)
    gamma = (torch.rand(64, generator=g) + 0.5).to(torch.bfloat16)
    sm = torch.rand(64, generator=g) + 0.5

    def block(x1, x2):
        y, _, x = torch.ops.npu.npu_add_rms_norm(x1, x2, gamma, 1e-5)
        q, s = torch.ops.npu.npu_dynamic_quant(y, smooth_scales=sm)
        return q, s, x

    gm = torch.fx.symbolic_trace(block)
    assert fuse_add_rms_norm_dynamic_quant(gm) == 1
    targets = {n.target for n in gm.graph.nodes if n.op == "call_function"}
    assert torch.ops.npu.npu_add_rms_norm_dynamic_quant.default in targets
    assert torch.ops.npu.npu_dynamic_quant.default not in targets
    for a, b in zip(gm(x1, x2), block(x1, x2)):
        assert torch.equal(a, b)
    fn = torch.compile(block, backend=get_npu_backend(), fullgraph=True)
    for a, b in zip(fn(x1, x2), block(x1, x2)):
        assert torch.equal(a, b)
    # rstd in use: no fusion of that call; a second call that only feeds a quant is fused
    def two(a, b):
        rstd = torch.ops.npu.npu_add_rms_norm(a, b, gamma)[1]
        q, s = torch.ops.npu.npu_dynamic_quant(torch.ops.npu.npu_add_rms_norm(a, b, gamma)[0])
        return rstd, q, s

    gm2 = torch.fx.symbolic_trace(two)
    assert fuse_add_rms_norm_dynamic_quant(gm2) == 1
    for a, b in zip(gm2(x1, x2), two(x1, x2)):
        assert torch.equal(a, b)


def test_pattern_pass_keeps_graph_order_when_x_out_is_used_before_the_quant():
    """A user of the norm's x output placed between the norm and the quant must still see a node
    defined before it (the fused node goes where the norm was)."""
    from oracle import cpu_ops
    from torchair_amd.patterns import fuse_add_rms_norm_dynamic_quant
    cpu_ops.register()
    g = torch.Generator().manual_seed(4)
    x1, x2 = torch.randn(4, 64, generator=g).to(torch.bfloat16), torch.randn(4, 64, generator=g).to(torch.bfloat16)
    gamma = (torch.rand(64, generator=g) + 0.5).to(torch.bfloat16)

    def block(x1, x2, sm):
        y, _, x = torch.ops.npu.npu_add_rms_norm(x1, x2, gamma)
        r = torch.relu(x)
        q, s = torch.ops.npu.npu_dynamic_quant(y, smooth_scales=sm * 2)  # smooth scale defined after the norm
        return q, s, r

    sm = torch.rand(64, generator=g) + 0.5
    gm = torch.fx.symbolic_trace(block)
    assert fuse_add_rms_norm_dynamic_quant(gm) == 0  # relu(x) precedes the smooth scale: left alone
    gm.graph.lint()

    def block2(x1, x2, sm):
        y, _, x = torch.ops.npu.npu_add_rms_norm(x1, x2, gamma)
        r = torch.relu(x)
        q, s = torch.ops.npu.npu_dynamic_quant(y, smooth_scales=sm)
        return q, s, r

    gm2 = torch.fx.symbolic_trace(block2)
    assert fuse_add_rms_norm_dynamic_quant(gm2) == 1
    gm2.graph.lint()
    for a, b in zip(gm2(x1, x2, sm), block2(x1, x2, sm)):
        assert torch.equal(a, b)


def test_pattern_pass_fuses_init_routing_dynamic_quant_on_cpu():
    """Routing whose expanded rows feed only a plain per-token quant becomes the routing op's quant
    mode 1; the compiled result equals the eager composition, bit for bit. A quant with smooth
    scales, or expanded rows with another user, is left alone."""
    from oracle import cpu_ops
    from torchair_amd.patterns import fuse_init_routing_dynamic_quant
    cpu_ops.register()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(16, 64, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(8, generator=g)[:2] for _ in range(16)]).to(torch.int32)
    sm = torch.rand(64, generator=g) + 0.5

    def block(x, idx):
        ex, ri, tok, _ = torch.ops.npu.npu_moe_init_routing_v2(x, idx, active_num=32, expert_num=8,
                                                               expert_tokens_num_type=1, expert_tokens_num_flag=True)
        q, s = torch.ops.npu.npu_dynamic_quant(ex)
        return q, s, ri, tok

    gm = torch.fx.symbolic_trace(block)
    assert fuse_init_routing_dynamic_quant(gm) == 1
    calls = [n for n in gm.graph.nodes if n.op == "call_function"]
    assert torch.ops.npu.npu_dynamic_quant.default not in {n.target for n in calls}
    assert [n.kwargs["quant_mode"] for n in calls if n.target == torch.ops.npu.npu_moe_init_routing_v2.default] == [1]
    for a, b in zip(gm(x, idx), block(x, idx)):
        assert torch.equal(a, b)
    fn = torch.compile(block, backend=get_npu_backend(), fullgraph=True)
    for a, b in zip(fn(x, idx), block(x, idx)):
        assert torch.equal(a, b)

    def smoothed(x, idx):
        ex, ri, tok, _ = torch.ops.npu.npu_moe_init_routing_v2(x, idx, expert_num=8)
        return torch.ops.npu.npu_dynamic_quant(ex, smooth_scales=sm)

    def rows_also_used(x, idx):
        ex, ri, tok, _ = torch.ops.npu.npu_moe_init_routing_v2(x, idx, expert_num=8)
        return torch.ops.npu.npu_dynamic_quant(ex), ex.float().sum()

    for f in (smoothed, rows_also_used):
        gm2 = torch.fx.symbolic_trace(f)
        assert fuse_init_routing_dynamic_quant(gm2) == 0
        gm2.graph.lint()


def test_pattern_pass_fuses_routing_into_grouped_matmul_on_cpu():
    """Dynamic-quant routing whose expanded rows feed only a grouped GEMM becomes the routing without
    the row copy plus a GEMM that gathers its rows; the compiled result equals the eager composition
    bit for bit (also with the routing's scales as the GEMM's per-token scales). Expanded rows with
    another user are left alone."""
    from oracle import cpu_ops
    from torchair_amd.patterns import fuse_init_routing_dynamic_quant, fuse_routing_grouped_matmul, stats
    cpu_ops.register()
    g = torch.Generator().manual_seed(7)
    t, h, e, k, n = 12, 64, 4, 2, 32
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
    w = torch.randint(-127, 128, (e, h, n), generator=g, dtype=torch.int8)
    ws = torch.rand(e, n, generator=g) * 0.01 + 1e-3
    npu = torch.ops.npu

    def block(x, idx):
        ex, ri, tok, _ = npu.npu_moe_init_routing_v2(x, idx, active_num=t * k, expert_num=e,
                                                     expert_tokens_num_type=1, expert_tokens_num_flag=True)
        q, s = npu.npu_dynamic_quant(ex)
        acc = npu.npu_grouped_matmul([q], [w], group_list=tok, split_item=3, group_type=0, group_list_type=1,
                                     output_dtype=torch.int32)[0]
        return acc, ri, tok

    def scaled(x, idx):
        q, ri, tok, s = npu.npu_moe_init_routing_v2(x, idx, active_num=t * k, expert_num=e, expert_tokens_num_type=1,
                                                    expert_tokens_num_flag=True, quant_mode=1)
        return npu.npu_grouped_matmul([q], [w], scale=[ws], per_token_scale=[s], group_list=tok, split_item=3,
                                      group_type=0, group_list_type=1, output_dtype=torch.bfloat16)[0], s

    for f, n_routes in ((block, 1), (scaled, 1)):
        gm = torch.fx.symbolic_trace(f)
        fuse_init_routing_dynamic_quant(gm)
        assert fuse_routing_grouped_matmul(gm) == n_routes
        targets = {nd.target for nd in gm.graph.nodes if nd.op == "call_function"}
        assert torch.ops.tai.grouped_matmul_gather.default in targets
        assert not {npu.npu_grouped_matmul, npu.npu_grouped_matmul.default} & targets
        for a, b in zip(gm(x, idx), f(x, idx)):
            assert torch.equal(a, b)
    before = stats["routing_grouped_matmul"]
    fn = torch.compile(block, backend=get_npu_backend(), fullgraph=True)
    for a, b in zip(fn(x, idx), block(x, idx)):
        assert torch.equal(a, b)
    assert stats["routing_grouped_matmul"] == before + 1

    ws = torch.rand(e, n, generator=g) * 0.01 + 1e-3

    def swiglu(x, idx):
        q, ri, tok, s = npu.npu_moe_init_routing_v2(x, idx, active_num=t * k, expert_num=e, expert_tokens_num_type=1,
                                                    expert_tokens_num_flag=True, quant_mode=1)
        acc = npu.npu_grouped_matmul([q], [w], group_list=tok, split_item=3, group_type=0, group_list_type=1,
                                     output_dtype=torch.int32)[0]
        return npu.npu_dequant_swiglu_quant(acc, weight_scale=ws, activation_scale=s, group_index=tok,
                                            activate_left=True, quant_mode=1)

    from torchair_amd.patterns import fuse_gather_dequant_swiglu_quant
    gm = torch.fx.symbolic_trace(swiglu)
    assert fuse_routing_grouped_matmul(gm) == 1 and fuse_gather_dequant_swiglu_quant(gm) == 1
    targets = {nd.target for nd in gm.graph.nodes if nd.op == "call_function"}
    assert torch.ops.tai.grouped_matmul_swiglu_quant_gather.default in targets
    assert not {npu.npu_dequant_swiglu_quant, npu.npu_dequant_swiglu_quant.default} & targets
    for a, b in zip(gm(x, idx), swiglu(x, idx)):
        assert torch.equal(a, b)

    def rows_also_used(x, idx):
        q, ri, tok, s = npu.npu_moe_init_routing_v2(x, idx, active_num=t * k, expert_num=e, expert_tokens_num_type=1,
                                                    expert_tokens_num_flag=True, quant_mode=1)
        acc = npu.npu_grouped_matmul([q], [w], group_list=tok, split_item=3, group_type=0, group_list_type=1,
                                     output_dtype=torch.int32)[0]
        return acc, q.sum()

    gm2 = torch.fx.symbolic_trace(rows_also_used)
    assert fuse_routing_grouped_matmul(gm2) == 0


def test_fia_dense_key_value_shapes_are_checked_before_launch():
    """Keys/values with fewer heads, another head dim or another batch than the query and
    num_key_value_heads declare are refused on the host (the kernels trust these sizes)."""
    from torchair_amd._fia import _dense_kv_check
    q = torch.zeros(2, 5, 8 * 64)
    good = torch.zeros(2, 7, 2 * 64)
    _dense_kv_check(q, good, good, "BSH", 8, 2)
    # too few heads, another batch, fewer value positions
    for k, v in ((torch.zeros(2, 7, 64), good), (torch.zeros(1, 7, 128), good), (good, torch.zeros(2, 6, 128))):
        with pytest.raises(RuntimeError):
            _dense_kv_check(q, k, v, "BSH", 8, 2)
    qn = torch.zeros(2, 8, 5, 64)
    _dense_kv_check(qn, torch.zeros(2, 2, 7, 64), torch.zeros(2, 2, 7, 64), "BNSD", 8, 2)
    with pytest.raises(RuntimeError):
        _dense_kv_check(qn, torch.zeros(2, 1, 7, 64), torch.zeros(2, 1, 7, 64), "BNSD", 8, 2)
    with pytest.raises(RuntimeError):
        _dense_kv_check(qn, torch.zeros(2, 2, 7, 32), torch.zeros(2, 2, 7, 64), "BNSD", 8, 2)
    qt = torch.zeros(9, 8, 64)
    _dense_kv_check(qt, torch.zeros(11, 2, 64), torch.zeros(11, 2, 64), "TND", 8, 2)
    _dense_kv_check(torch.zeros(8, 9, 64), torch.zeros(2, 11, 64), torch.zeros(2, 11, 64), "NTD", 8, 2)
    with pytest.raises(RuntimeError):
        _dense_kv_check(qt, torch.zeros(11, 1, 64), torch.zeros(11, 1, 64), "TND", 8, 2)
    with pytest.raises(RuntimeError):
        _dense_kv_check(qt, torch.zeros(11, 2, 64), torch.zeros(10, 2, 64), "TND", 8, 2)


def test_fia_host_helpers_for_packed_layouts_and_quant_scales():
    """Host logic of the packed layouts and the int8 query, without a GPU: which TND calls keep the
    one-token kernels, the longest run of cumulative ends, and UINT64 scales carrying an fp32 in their
    low 32 bits."""
    from torchair_amd._fia import _max_run, _one_scale, _one_token_each
    q = torch.zeros(4, 2, 64)
    assert _one_token_each(q, "TND", "TND", {}, 4)
    assert _one_token_each(q, "TND", "TND", {"actual_seq_lengths": [1, 2, 3, 4]}, 4)
    assert not _one_token_each(q, "TND", "TND", {"actual_seq_lengths": [1, 2, 4, 4]}, 4)
    assert not _one_token_each(q, "TND", "TND", {"actual_seq_lengths": torch.arange(1, 5)}, 4)  # device values
    assert not _one_token_each(q, "TND", "NTD", {}, 4) and not _one_token_each(q, "TND", "TND", {}, 3)
    assert _max_run(torch.tensor([3, 3, 10, 12])) == 7 and _max_run(torch.tensor([], dtype=torch.int64)) == 0
    f = np.float32(0.0123)
    bits = int(np.array([f]).view(np.uint32)[0]) | (5 << 40)  # high bits are not part of the scale
    for t in (torch.tensor([bits], dtype=torch.int64), torch.tensor([0.0123], dtype=torch.float32)):
        got = _one_scale(t, "dequant_scale1")
        assert got.dtype == torch.float32 and got.numel() == 1 and got.item() == float(f)
    with pytest.raises(RuntimeError, match="one"):
        _one_scale(torch.ones(2), "quant_scale1")


def test_ops_alias_exposes_the_reference_entry_points():
    """torchair_amd.ops carries the fused-op functions of the reference's torchair.ops for this path."""
    from torchair_amd import ops
    for name in ("npu_fused_infer_attention_score", "npu_fused_infer_attention_score_v2"):
        assert callable(getattr(ops, name))
    assert ops.npu_dynamic_quant is torch.ops.npu.npu_dynamic_quant
    # every npu:: op this package defines is reachable through the alias
    import re
    src = "".join((ROOT / "torchair_amd" / f).read_text() for f in ("_ops_impl.py", "_norm_cache.py", "_gmm_fused.py"))
    for name in set(re.findall(r'"(npu_[a-z0-9_]+)\(', src)):
        assert hasattr(ops, name), name
