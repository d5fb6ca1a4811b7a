"""FX fusion passes applied before lowering (CompilerConfig.experimental_config.pattern_fusion_pass).

add_rms_norm + dynamic_quant -> add_rms_norm_dynamic_quant, the rewrite of
python/torchair/patterns/add_rms_norm_dynamic_quant.py:67-80 (and its epsilon / no-x-out
variants): npu_add_rms_norm(x1, x2, gamma[, eps]) whose normalised output feeds only
npu_dynamic_quant(y, smooth_scales=s) becomes npu_add_rms_norm_dynamic_quant(x1, x2, gamma,
smooth_scale1=s, epsilon=eps, output_mask=[True, False]); the fused kernel quantises y rounded to
the input dtype, so the rewrite changes no value. A match whose rstd output is used, or whose
quant has other arguments than smooth_scales, is left alone.

npu_moe_init_routing_v2 + dynamic_quant -> npu_moe_init_routing_v2(quant_mode=1): routing without
quantisation whose expanded rows feed only a symmetric per-token int8 npu_dynamic_quant (no smooth
scales, no group index) becomes the routing op with its dynamic quant mode (experiment_ops.h:2167),
whose expanded rows and scales are the quantised rows and their scales. The routing kernel quantises
each token row once and gathers the int8 rows, which equals quantising every gathered copy, so the
rewrite changes no value. This pattern has no counterpart among the reference's passes.

npu_moe_init_routing_v2(quant_mode=1) + npu_grouped_matmul -> tai::moe_init_routing_v2_rows +
tai::grouped_matmul_gather: dynamic-quant routing (dropless, no smooth scale) whose expanded rows feed
only the x of a grouped GEMM (groups along M, one output) becomes the routing without the copy of the
rows, and the GEMM reads each product row from the quantised token rows through the routing's row map
(the same int8 bytes, so the rewrite changes no value; at DeepSeek-V3 decode shapes it saves writing
and re-reading T * k rows). This pattern has no counterpart among the reference's passes.
"""
from __future__ import annotations

import logging
import operator

import torch
import torch.fx

logger = logging.getLogger("torchair_amd")

# rewrites applied so far in this process, per pattern (diagnostics and tests)
stats = {"add_rms_norm_dynamic_quant": 0, "init_routing_dynamic_quant": 0, "routing_grouped_matmul": 0,
         "gather_dequant_swiglu_quant": 0}


def _getitems(node: torch.fx.Node):
    """index -> list of getitem users of a multi-output node; None if another kind of use exists."""
    out = {}
    for u in node.users:
        if u.op != "call_function" or u.target is not operator.getitem:
            return None
        out.setdefault(u.args[1], []).append(u)
    return out


def _calls(node: torch.fx.Node, packet) -> bool:
    """True for a call of the op (its packet, as symbolic tracing records it, or its default overload)."""
    return node.op == "call_function" and node.target in (packet, packet.default)


def fuse_add_rms_norm_dynamic_quant(gm: torch.fx.GraphModule) -> int:
    npu = torch.ops.npu
    if not hasattr(npu, "npu_add_rms_norm_dynamic_quant"):
        return 0
    fused = 0
    for norm in list(gm.graph.nodes):
        if not _calls(norm, npu.npu_add_rms_norm):
            continue
        outs = _getitems(norm)
        if outs is None:
            continue
        dead = [u for us in outs.values() for u in us if not u.users]
        outs = {i: [u for u in us if u.users] for i, us in outs.items()}
        if outs.get(1) or len(outs.get(0, [])) != 1:
            continue
        y = outs[0][0]
        if len(y.users) != 1:
            continue
        quant = next(iter(y.users))
        if not _calls(quant, npu.npu_dynamic_quant):
            continue
        if quant.args[0] is not y or len(quant.args) != 1 or set(quant.kwargs) - {"smooth_scales"}:
            continue
        qouts = _getitems(quant)
        if qouts is None:
            continue
        # the fused node takes the norm's place, or the smooth scale's when that is defined later;
        # users of the norm's x output must all come after that point
        order = {n: i for i, n in enumerate(gm.graph.nodes)}
        smooth = quant.kwargs.get("smooth_scales")
        anchor = smooth if isinstance(smooth, torch.fx.Node) and order[smooth] > order[norm] else norm
        if any(order[u] <= order[anchor] for xu in outs.get(2, []) for u in xu.users):
            continue
        for us in qouts.values():
            for u in [u for u in us if not u.users]:
                us.remove(u)
                gm.graph.erase_node(u)
        x1, x2, gamma = norm.args[:3]
        eps = norm.args[3] if len(norm.args) > 3 else norm.kwargs.get("epsilon", 1e-6)
        with gm.graph.inserting_after(anchor):
            node = gm.graph.call_function(
                npu.npu_add_rms_norm_dynamic_quant.default, (x1, x2, gamma),
                {"smooth_scale1": quant.kwargs.get("smooth_scales"), "epsilon": eps, "output_mask": [True, False]})
        for src_idx, users, dst_idx in ((0, qouts.get(0, []), 0), (1, qouts.get(1, []), 3), (2, outs.get(2, []), 2)):
            for u in users:
                with gm.graph.inserting_after(node):
                    new = gm.graph.call_function(operator.getitem, (node, dst_idx))
                u.replace_all_uses_with(new)
                gm.graph.erase_node(u)
        gm.graph.erase_node(quant)
        gm.graph.erase_node(y)
        for u in dead:
            gm.graph.erase_node(u)
        gm.graph.erase_node(norm)
        fused += 1
    if fused:
        gm.graph.lint()
        gm.recompile()
        stats["add_rms_norm_dynamic_quant"] += fused
        logger.debug("fused %d add_rms_norm + dynamic_quant pair(s)", fused)
    return fused


def _plain_dynamic_quant(quant: torch.fx.Node, rows: torch.fx.Node) -> bool:
    """npu_dynamic_quant(rows) as symmetric per-token int8 without smooth scales or groups."""
    if quant.args != (rows,):
        return False
    kw = dict(quant.kwargs)
    ok = {"smooth_scales": (None,), "group_index": (None,), "dst_type": (None, 1, torch.int8),
          "quant_mode": (None, "pertoken"), "dst_type_max": (None, 0.0)}
    return all(k in ok and any(v is a or v == a for a in ok[k]) for k, v in kw.items())


def fuse_init_routing_dynamic_quant(gm: torch.fx.GraphModule) -> int:
    npu = torch.ops.npu
    if not hasattr(npu, "npu_moe_init_routing_v2"):
        return 0
    fused = 0
    for route in list(gm.graph.nodes):
        if not _calls(route, npu.npu_moe_init_routing_v2) or len(route.args) != 2:
            continue
        kw = dict(route.kwargs)
        if kw.get("quant_mode", -1) != -1 or kw.get("scale") is not None or kw.get("offset") is not None:
            continue
        outs = _getitems(route)
        if outs is None:
            continue
        live = {i: [u for u in us if u.users] for i, us in outs.items()}
        if live.get(3) or len(live.get(0, [])) != 1:
            continue
        rows = live[0][0]
        if len(rows.users) != 1:
            continue
        quant = next(iter(rows.users))
        if not _calls(quant, npu.npu_dynamic_quant) or not _plain_dynamic_quant(quant, rows):
            continue
        qouts = _getitems(quant)
        if qouts is None:
            continue
        kw["quant_mode"] = 1
        with gm.graph.inserting_after(route):
            node = gm.graph.call_function(npu.npu_moe_init_routing_v2.default, route.args, kw)
        # quant outputs 0 / 1 become the routing's expanded rows / expanded scales; its other outputs
        # move over unchanged
        for users, dst_idx in ((qouts.get(0, []), 0), (qouts.get(1, []), 3), (outs.get(1, []), 1), (outs.get(2, []), 2)):
            for u in users:
                with gm.graph.inserting_after(node):
                    new = gm.graph.call_function(operator.getitem, (node, dst_idx))
                u.replace_all_uses_with(new)
                gm.graph.erase_node(u)
        gm.graph.erase_node(quant)
        for us in outs.values():
            for u in us:
                if u in gm.graph.nodes and not u.users:
                    gm.graph.erase_node(u)
        gm.graph.erase_node(route)
        fused += 1
    if fused:
        gm.graph.lint()
        gm.recompile()
        stats["init_routing_dynamic_quant"] += fused
        logger.debug("fused %d init_routing_v2 + dynamic_quant pair(s)", fused)
    return fused


def _gather_gmm_kwargs(gmm: torch.fx.Node, rows: torch.fx.Node):
    """kwargs of tai::grouped_matmul_gather for npu_grouped_matmul([rows], [w], ...) with groups along M,
    one output over all rows and nothing the gather op does not take; None otherwise."""
    if len(gmm.args) != 2 or not all(isinstance(a, (list, tuple)) and len(a) == 1 for a in gmm.args):
        return None
    if gmm.args[0][0] is not rows or gmm.args[1][0] is rows:
        return None
    kw = dict(gmm.kwargs)
    if not isinstance(kw.get("group_list"), torch.fx.Node) or kw.get("group_list_type", 0) not in (0, 1):
        return None
    if kw.get("split_item") not in (2, 3) or kw.get("group_type") not in (None, 0) or kw.get("act_type") not in (None, 0):
        return None
    out = {"group_list_type": kw.get("group_list_type", 0), "output_dtype": kw.get("output_dtype")}
    for name in ("scale", "per_token_scale", "bias"):
        v = kw.get(name)
        if v is None or (isinstance(v, (list, tuple)) and not v):
            continue
        if not (isinstance(v, (list, tuple)) and len(v) == 1 and isinstance(v[0], torch.fx.Node)):
            return None
        out[name] = v[0]
    free = {"group_list", "group_list_type", "split_item", "group_type", "act_type", "output_dtype", "tuning_config",
            "scale", "per_token_scale", "bias"}
    if any(not (v is None or (isinstance(v, (list, tuple)) and not v)) for k, v in kw.items() if k not in free):
        return None
    return out


def fuse_routing_grouped_matmul(gm: torch.fx.GraphModule) -> int:
    npu, tai = torch.ops.npu, getattr(torch.ops, "tai", None)
    if tai is None or not hasattr(tai, "grouped_matmul_gather") or not hasattr(npu, "npu_moe_init_routing_v2"):
        return 0
    fused = 0
    for route in list(gm.graph.nodes):
        if not _calls(route, npu.npu_moe_init_routing_v2) or len(route.args) != 2:
            continue
        kw = dict(route.kwargs)
        if kw.get("quant_mode") != 1 or kw.get("scale") is not None or kw.get("offset") is not None:
            continue
        if kw.get("drop_pad_mode", 0) not in (0, None):
            continue
        allowed = {"quant_mode", "scale", "offset", "drop_pad_mode", "active_num", "expert_num", "expert_capacity",
                   "expert_tokens_num_type", "expert_tokens_num_flag", "active_expert_range", "row_idx_type"}
        if set(kw) - allowed:
            continue
        outs = _getitems(route)
        if outs is None:
            continue
        live0 = [u for u in outs.get(0, []) if u.users]
        if len(live0) != 1 or len(live0[0].users) != 1:
            continue
        rows = live0[0]
        gmm = next(iter(rows.users))
        if not _calls(gmm, npu.npu_grouped_matmul):
            continue
        gkw = _gather_gmm_kwargs(gmm, rows)
        gouts = _getitems(gmm) if gkw is not None else None
        if gouts is None or set(gouts) - {0}:
            continue
        rkw = {k: kw[k] for k in ("active_num", "expert_num", "expert_tokens_num_type", "row_idx_type") if k in kw}
        if kw.get("active_expert_range"):
            rkw["active_expert_range"] = list(kw["active_expert_range"])
        with gm.graph.inserting_after(route):
            node = gm.graph.call_function(tai.moe_init_routing_v2_rows.default, route.args, rkw)
        with gm.graph.inserting_after(node):
            q = gm.graph.call_function(operator.getitem, (node, 0))
        with gm.graph.inserting_after(q):
            a_rows = gm.graph.call_function(operator.getitem, (node, 1))
        # the routing's other outputs move over: row index, token counts, scales
        for src_idx, dst_idx in ((1, 2), (2, 3), (3, 4)):
            for u in outs.get(src_idx, []):
                with gm.graph.inserting_after(a_rows):
                    new = gm.graph.call_function(operator.getitem, (node, dst_idx))
                u.replace_all_uses_with(new)
                gm.graph.erase_node(u)
        gkw = _gather_gmm_kwargs(gmm, rows)  # again: operands that were routing outputs moved over
        with gm.graph.inserting_before(gmm):
            gnode = gm.graph.call_function(tai.grouped_matmul_gather.default,
                                           (q, a_rows, gmm.args[1][0], gmm.kwargs["group_list"]), gkw)
        for u in gouts.get(0, []):
            u.replace_all_uses_with(gnode)
            gm.graph.erase_node(u)
        gm.graph.erase_node(gmm)
        for u in outs.get(0, []):
            gm.graph.erase_node(u)
        gm.graph.erase_node(route)
        fused += 1
    if fused:
        gm.graph.lint()
        gm.recompile()
        stats["routing_grouped_matmul"] += fused
        logger.debug("fused %d init_routing_v2 + grouped_matmul pair(s)", fused)
    return fused


def fuse_gather_dequant_swiglu_quant(gm: torch.fx.GraphModule) -> int:
    tai, npu = getattr(torch.ops, "tai", None), torch.ops.npu
    if tai is None or not hasattr(tai, "grouped_matmul_swiglu_quant_gather"):
        return 0
    fused = 0
    for gmm in list(gm.graph.nodes):
        if not _calls(gmm, tai.grouped_matmul_gather) or len(gmm.args) != 4 or len(gmm.users) != 1:
            continue
        kw = dict(gmm.kwargs)
        if kw.get("output_dtype") not in (torch.int32, 3) or kw.get("group_list_type") != 1:
            continue
        if any(kw.get(k) is not None for k in ("scale", "per_token_scale", "bias")):
            continue
        dsq = next(iter(gmm.users))
        if not _calls(dsq, npu.npu_dequant_swiglu_quant) or dsq.args != (gmm,):
            continue
        dkw = dict(dsq.kwargs)
        counts = gmm.args[3]
        ok = {"weight_scale", "activation_scale", "group_index", "activate_left", "quant_mode", "dst_type",
              "round_mode", "activate_dim", "swiglu_mode", "bias", "quant_scale", "quant_offset"}
        if set(dkw) - ok or dkw.get("group_index") is not counts or dkw.get("activate_left") is not True:
            continue
        if dkw.get("quant_mode") != 1 or dkw.get("dst_type") not in (None, 1) or dkw.get("round_mode") not in (None, 0):
            continue
        if dkw.get("activate_dim") not in (None, -1, 1) or dkw.get("swiglu_mode", 0) != 0:
            continue
        if any(dkw.get(k) is not None for k in ("bias", "quant_scale", "quant_offset")):
            continue
        if not isinstance(dkw.get("weight_scale"), torch.fx.Node) or not isinstance(dkw.get("activation_scale"),
                                                                                     torch.fx.Node):
            continue
        x, a_rows, w = gmm.args[:3]
        with gm.graph.inserting_before(dsq):
            node = gm.graph.call_function(tai.grouped_matmul_swiglu_quant_gather.default,
                                          (x, a_rows, w, dkw["weight_scale"], dkw["activation_scale"], counts),
                                          {"group_list_type": 1})
        dsq.replace_all_uses_with(node)  # both return (y, scale)
        gm.graph.erase_node(dsq)
        gm.graph.erase_node(gmm)
        fused += 1
    if fused:
        gm.graph.lint()
        gm.recompile()
        stats["gather_dequant_swiglu_quant"] += fused
        logger.debug("fused %d grouped_matmul_gather + dequant_swiglu_quant pair(s)", fused)
    return fused


def apply_pattern_passes(gm: torch.fx.GraphModule) -> torch.fx.GraphModule:
    fuse_add_rms_norm_dynamic_quant(gm)
    fuse_init_routing_dynamic_quant(gm)
    fuse_routing_grouped_matmul(gm)
    fuse_gather_dequant_swiglu_quant(gm)
    return gm
