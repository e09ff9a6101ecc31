"""Graph passes of the MI355X pipeline.

Same pass sequence and semantics as the reference's default pipelines
(passes/base.py:67-161) for the parts that decide what the device executes:

  O0   liveness -> memory plan
  O1   identity elimination -> dead-code elimination -> liveness -> plan
  O2   as O1; at any level a max_memory below the plan's peak is met by
       spilling tensors to pinned host memory and reloading them before
       their next use (fit_memory)
  O3   O1 + pattern fusion (conv_relu, conv_sigmoid, add_relu, add_sigmoid,
       matmul_relu; pattern/fusion_patterns.py:105-153) + prepack lowering
       (conv kernel kind, constant Gemm B transposed to [N, K];
       passes/prepack_lowering.py:48-118)

The memory plan places every non-constant tensor at an offset of one HBM
arena, reusing the space of tensors whose last use has passed, and lets the
element-wise ops write over an input that dies at that node, like the
reference's cost_aware strategy (passes/strategies/cost_aware_allocator.py:
39-48, 412-436). Constants get their own region of the same arena.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .ir import Graph, Node, TensorInfo

ALIGN = 256  # arena offsets; 16-byte vector loads need 16, 256 keeps rows cache-line aligned

# ops that may write over a same-sized input that dies at the node
# (cost_aware_allocator.py:39-48)
INPLACE_OPS = {"Relu", "Sigmoid", "Tanh", "Add", "Sub", "Mul", "Div", "Clip",
               "FusedAddRelu", "FusedAddSigmoid", "FusedConvAddRelu", "FusedEltwise"}
# inputs an in-place output may take over (default: any); the fused conv
# reads its image input at neighbouring pixels, so only the residual
INPLACE_INPUTS = {"FusedConvAddRelu": (3,)}


# ---------------------------------------------------------------------------
# cleanup
# ---------------------------------------------------------------------------
def eliminate_identity(g: Graph) -> int:
    """Bypass Identity nodes (passes/identity_elimination.py:13): consumers read
    the Identity's input. An Identity producing a graph output is kept."""
    removed = 0
    for node in list(g.nodes):
        if node.op_type != "Identity" or node.outputs[0] in g.outputs:
            continue
        src, dst = node.inputs[0], node.outputs[0]
        for c in g.nodes:
            c.inputs = [src if i == dst else i for i in c.inputs]
        g.nodes.remove(node)
        g.tensors.pop(dst, None)
        removed += 1
    return removed


def eliminate_dead_code(g: Graph) -> int:
    """Drop nodes none of whose outputs reach a graph output
    (passes/dead_code_elimination.py:13), then unreferenced tensors."""
    live = set(g.outputs)
    keep = []
    for node in reversed(g.topological_sort()):
        if any(o in live for o in node.outputs):
            keep.append(node)
            live.update(i for i in node.inputs if i)
    removed = len(g.nodes) - len(keep)
    kept = set(id(n) for n in keep)
    g.nodes = [n for n in g.nodes if id(n) in kept]
    used = set(g.inputs) | set(g.outputs)
    for n in g.nodes:
        used.update(n.inputs)
        used.update(n.outputs)
    for name in list(g.tensors):
        if name not in used:
            del g.tensors[name]
    return removed


# ---------------------------------------------------------------------------
# pattern fusion (O3)
# ---------------------------------------------------------------------------
_PATTERNS = [  # (producer, consumer, fused op), in priority order
    ("Conv", "Relu", "FusedConvRelu"),
    ("Conv", "Sigmoid", "FusedConvSigmoid"),
    ("Add", "Relu", "FusedAddRelu"),
    ("Add", "Sigmoid", "FusedAddSigmoid"),
    ("MatMul", "Relu", "FusedMatMulRelu"),
]


def fuse_patterns(g: Graph) -> int:
    """producer().only_used_by(consumer()) -> one fused node carrying the
    producer's inputs/attrs and the consumer's output."""
    fused = 0
    for prod_op, cons_op, fused_op in _PATTERNS:
        for node in list(g.nodes):
            if node.op_type != prod_op or node.outputs[0] in g.outputs:
                continue
            users = g.consumers(node.outputs[0])
            if len(users) != 1 or users[0].op_type != cons_op:
                continue
            user = users[0]
            mid = node.outputs[0]
            node.op_type = fused_op
            node.outputs = list(user.outputs)
            node.metadata["fused_from"] = [node.name, user.name]
            g.nodes.remove(user)
            g.tensors.pop(mid, None)
            fused += 1
    return fused


def fuse_residual(g: Graph) -> int:
    """mi355x target, O3: a fused Add+Relu one of whose operands is produced
    by a Conv (no activation) used only there, the other operand having the
    conv output's exact shape, becomes one FusedConvAddRelu node (inputs: x,
    w, bias or "", residual), lowered to nnc_hip_conv_add_relu: the residual
    is added in the conv epilogue instead of a separate pass over both
    tensors. The Add's first operand is preferred (the block's main-path
    conv in ResNet; the shortcut conv stays a plain conv)."""
    fused = 0
    for add in list(g.nodes):
        if add.op_type != "FusedAddRelu" or len(add.inputs) != 2 or add.inputs[0] == add.inputs[1]:
            continue
        for k in (0, 1):
            mid, res = add.inputs[k], add.inputs[1 - k]
            prod = g.producer(mid)
            if prod is None or prod.op_type != "Conv" or mid in g.outputs:
                continue
            if len(g.consumers(mid)) != 1:
                continue
            if g.tensors[res].shape != g.tensors[mid].shape or g.tensors[res].dtype != g.tensors[mid].dtype:
                continue
            inputs = list(prod.inputs) + [""] * (3 - len(prod.inputs))
            prod.inputs = inputs[:3] + [res]
            prod.op_type = "FusedConvAddRelu"
            prod.outputs = list(add.outputs)
            prod.metadata["fused_from"] = [prod.name, add.name]
            g.nodes.remove(add)
            g.tensors.pop(mid, None)
            fused += 1
            break
    return fused


CONV_OPS = ("Conv", "FusedConvRelu", "FusedConvSigmoid", "FusedConvAddRelu")
# every node that runs a convolution, for FLOP accounting (the projection
# conv's packed [Co][9*Ci + Cx] weight gives its K)
FLOP_CONV_OPS = CONV_OPS + ("FusedConvProjRelu",)


def pack_conv_weights(g: Graph) -> int:
    """mi355x target, O3: convolutions whose weight is a constant used only
    there get the weight transposed at compile time to tap-major order and
    are lowered to nnc_hip_conv_packed, whose kernels stream that layout
    straight into LDS: 3x3 kernels with Ci % 32 == 0 as [Co][kh][kw][Ci],
    the 3-channel 7x7 stem as [Co][Kp] (rows of K = 147 tap-major values
    zero-padded to 160). 1x1 weights already have the tap-major layout and
    keep their reference entry points (which take the same kernels)."""
    packed = 0
    for node in g.nodes:
        if node.op_type not in CONV_OPS or len(node.inputs) < 2:
            continue
        wname = node.inputs[1]
        w = g.tensors[wname]
        x = g.tensors[node.inputs[0]]
        if not w.is_constant or w.data is None or w.data.ndim != 4 or len(g.consumers(wname)) != 1:
            continue
        co, ci, kh, kw = w.data.shape
        if len(x.shape) != 4 or x.shape[1] != ci:
            continue
        if int(node.attrs.get("group", 1)) != 1 or list(node.attrs.get("dilations", [1, 1])) != [1, 1]:
            continue
        tap_major = w.data.transpose(0, 2, 3, 1)
        if (kh, kw) == (7, 7) and ci == 3:
            k = kh * kw * ci
            rows = np.zeros((co, (k + 31) // 32 * 32), w.data.dtype)
            rows[:, :k] = tap_major.reshape(co, k)
            w.data = rows
        elif (kh, kw) == (3, 3) and ci % 32 == 0:
            w.data = np.ascontiguousarray(tap_major)
        else:
            continue
        w.shape = tuple(w.data.shape)
        node.attrs["kernel_shape"] = [kh, kw]
        node.metadata.setdefault("lowering", {})["weight_pack"] = "tap_major"
        packed += 1
    return packed


def fuse_projection(g: Graph) -> int:
    """mi355x target, O3, after pack_conv_weights: a residual block whose
    shortcut is a 1x1 convolution P (constant weights, no padding, output
    read only by the block's last convolution F, a packed 3x3
    FusedConvAddRelu) becomes one FusedConvProjRelu node lowered to
    nnc_hip_conv_proj: P's weights are appended to each packed row of F's
    ([Co][9*Ci + Cx]), the two biases summed, and P's input read by F's
    contraction, so the projection needs no launch and no tensor. Inputs:
    x, w, bias or "", projection input; attrs: F's, plus proj_strides."""
    fused = 0
    for f in list(g.nodes):
        if f.op_type != "FusedConvAddRelu" or len(f.inputs) != 4:
            continue
        if f.metadata.get("lowering", {}).get("weight_pack") != "tap_major":
            continue
        h, wname, bname, res = f.inputs
        wf = g.tensors[wname]
        if wf.data is None or wf.data.ndim != 4 or wf.data.shape[1:3] != (3, 3):
            continue
        p = g.producer(res)
        if p is None or p.op_type != "Conv" or res in g.outputs or len(g.consumers(res)) != 1:
            continue
        if len(p.inputs) < 2 or not g.tensors[p.inputs[1]].is_constant or len(g.consumers(p.inputs[1])) != 1:
            continue
        wp = g.tensors[p.inputs[1]].data
        x = g.tensors[p.inputs[0]]
        if wp is None or wp.ndim != 4 or wp.shape[2:] != (1, 1) or len(x.shape) != 4:
            continue
        if list(p.attrs.get("pads", [0, 0, 0, 0])) != [0, 0, 0, 0] or int(p.attrs.get("group", 1)) != 1:
            continue
        if list(p.attrs.get("dilations", [1, 1])) != [1, 1] or g.tensors[res].shape != g.tensors[f.outputs[0]].shape:
            continue
        co, ci, cx = wf.data.shape[0], wf.data.shape[3], wp.shape[1]
        if wp.shape[0] != co or ci % 32 or cx % 32:
            continue
        biases = [n for n in (bname, p.inputs[2] if len(p.inputs) > 2 else "") if n]
        if any(not g.tensors[n].is_constant or len(g.consumers(n)) != 1 for n in biases):
            continue
        rows = np.concatenate([wf.data.reshape(co, 9 * ci), wp.reshape(co, cx)], axis=1)
        w_new = _fresh(g.tensors, f"{wname}.proj")
        g.add_tensor(TensorInfo(w_new, tuple(rows.shape), wf.dtype, np.ascontiguousarray(rows)))
        b_new = ""
        if biases:
            total = np.zeros(co, np.float32)
            for n in biases:
                total = total + g.tensors[n].data.reshape(co).astype(np.float32)
            b_new = _fresh(g.tensors, f"{bname or biases[0]}.proj")
            g.add_tensor(TensorInfo(b_new, (co,), "float32", total.astype(np.float32)))
        f.metadata["weights_from"] = [wname, p.inputs[1]]
        for n in [wname, p.inputs[1]] + biases:
            g.tensors.pop(n, None)
        f.inputs = [h, w_new, b_new, p.inputs[0]]
        f.op_type = "FusedConvProjRelu"
        f.attrs["proj_strides"] = list(p.attrs.get("strides", [1, 1]))
        f.metadata["fused_from"] = f.metadata.get("fused_from", [f.name]) + [p.name]
        g.nodes.remove(p)
        g.tensors.pop(res, None)
        fused += 1
    return fused


def fuse_matmul_bias(g: Graph) -> int:
    """mi355x target, O3: MatMul(activation, constant W [K, N]) whose only
    consumer adds a constant 1-D bias [N] becomes one GEMM with the bias in
    its epilogue: FusedMatMulBias (lowered to nnc_gemm_nt on [M, K] / [M, N]
    views, W packed to [N, K] at compile time) or, when the Add was fused
    with a Relu, FusedMatMulBiasRelu (lowered to nnc_matmul_relu with the
    bias). The sum is the same fp32 add of the bias to the product."""
    fused = 0
    for mm in list(g.nodes):
        if mm.op_type != "MatMul" or len(mm.inputs) != 2 or mm.outputs[0] in g.outputs:
            continue
        a, w = mm.inputs
        wt = g.tensors[w]
        if not wt.is_constant or len(wt.shape) != 2 or len(g.tensors[a].shape) < 2:
            continue
        mid = mm.outputs[0]
        users = g.consumers(mid)
        if len(users) != 1 or users[0].op_type not in ("Add", "FusedAddRelu") or len(users[0].inputs) != 2:
            continue
        add = users[0]
        bias = add.inputs[1] if add.inputs[0] == mid else add.inputs[0]
        bt = g.tensors[bias]
        n = wt.shape[1]
        if bias == mid or not bt.is_constant or tuple(bt.shape) != (n,):
            continue
        relu = add.op_type == "FusedAddRelu"
        if not relu and len(g.consumers(w)) == 1:
            wt.data = np.ascontiguousarray(wt.data.T)
            wt.shape = tuple(wt.data.shape)
            mm.attrs["transB"] = 1
        elif not relu:
            continue  # a shared weight keeps its layout; leave the pair unfused
        mm.op_type = "FusedMatMulBiasRelu" if relu else "FusedMatMulBias"
        mm.inputs = [a, w, bias]
        mm.outputs = list(add.outputs)
        mm.metadata["fused_from"] = [mm.name, add.name]
        g.nodes.remove(add)
        g.tensors.pop(mid, None)
        fused += 1
    return fused


def prepack_lowering(g: Graph) -> None:
    """Conv kernel kind and constant Gemm B packing
    (passes/prepack_lowering.py:48-118)."""
    for node in g.nodes:
        if node.op_type in CONV_OPS:
            kh, kw = node.attrs.get("kernel_shape", [1, 1])
            sh, sw = node.attrs.get("strides", [1, 1])
            pads = node.attrs.get("pads", [0, 0, 0, 0])
            ph, pw = pads[0], pads[1]
            kind = "generic"
            if kh == 1 and kw == 1:
                kind = "pointwise_1x1"
            elif (kh, kw, sh, sw, ph, pw) == (3, 3, 1, 1, 1, 1):
                kind = "spatial_3x3"
            elif (kh, kw, sh, sw, ph, pw) == (7, 7, 2, 2, 3, 3):
                kind = "stem_7x7_s2"
            node.metadata.setdefault("lowering", {})["kernel_kind"] = kind
        elif node.op_type == "Gemm" and len(node.inputs) >= 2:
            low = node.metadata.setdefault("lowering", {})
            wname = node.inputs[1]
            w = g.tensors[wname]
            if int(node.attrs.get("transA", 0)) != 0:
                continue
            if int(node.attrs.get("transB", 0)) == 1:
                if w.is_constant:
                    low["weight_pack"] = "rhs_transposed_constant"
                continue
            if w.is_constant and w.data.ndim == 2 and len(g.consumers(wname)) == 1:
                w.data = np.ascontiguousarray(w.data.T)
                w.shape = tuple(w.data.shape)
                node.attrs["transB"] = 1
                low["weight_pack"] = "rhs_transposed_constant"


# ---------------------------------------------------------------------------
# tile streaming between ops (mi355x O3): the tiling half of the reference's
# O3 pipeline, ScheduleAnalysis -> LayoutPlanning -> TiledLowering
# (passes/base.py:113-124), re-targeted from x86 fast memory to a GPU
# workgroup's on-chip memory
# ---------------------------------------------------------------------------
# The reference schedules ops whose working set fits a 1 MiB fast memory
# (schedule_analysis.py:12) and streams their tiles through it
# (tiled_lowering.py:44-759). On the MI355X the fast memory of a producer's
# tile is the workgroup's LDS (128 KiB here, of the CU's 160 KiB) and its
# registers: a producer -> consumer pair is streamed when the consumer needs
# only what one workgroup of the fused kernel computes and that fits this
# budget, and the intermediate tensor then never exists in HBM.
LDS_BUDGET = 128 * 1024
# The fused GAP -> Gemm kernel re-reads an image's planes for every group of
# 16 classes and serialises its loads, means and dot products in one
# workgroup, so it can only pay where the unfused pair is two launches of
# little work. Measured on MI355X with ResNet-18's classifier (hipGraph
# replay of the whole network, hipEvent kernel times): fused 16.4 / 17.4 /
# 16.9 / 29.4 us at batch 1 / 2 / 4 / 8 against GAP + classifier 12.4 /
# 21.9 / 23.6 / 21.8 us, whole steps 0.2704 vs 0.2628 ms at batch 1, equal
# at 2 and 4, 0.598 vs 0.586 ms at 8. It is taken up to this batch: none by
# default, the pass and the kernel stay for programs where it pays.
GAP_GEMM_MAX_BATCH = 0

# LDS of the fused GAP -> Gemm kernel (nnc_hip_gap_gemm_nt) per workgroup:
# one image's planes and its C means (its rows of w are in registers)
def gap_gemm_lds_bytes(channels: int, plane: int) -> int:
    return 4 * (channels + channels * (plane + 1))


# The stem streamed into its max pool (nnc_hip_conv_maxpool). On the stem
# row kernel's shapes (224x224 or 64x64 RGB, stride 2, pad 3) with at least
# two conv rows per CU the library pools inside that kernel, bit-identical
# to the unfused pair; measured on MI355X (ResNet-18's stem conv + max pool):
# fused 94.5 / 36.1 / 34.2 us at batch 32 / 8 / 5 against 115.3 / 42.7 / 36.6
# us unfused. Elsewhere it runs a 64x128-tile kernel that measured slower
# than the pair (35.4 / 57.6 us at batch 1 / 8 against 15.1 / 53.6 us).
# Fused from this many conv output rows (N x Ho) on the row kernel's shapes:
# two rows per CU of MI355X's 256, the row kernel's own floor (batch 5 at
# 224x224); None: never (1: always, any shape the entry point takes).
CONV_POOL_MIN_ROWS: int | None = 512


def conv_pool_lds_bytes(wo: int | None = None) -> int:
    """LDS of the fused stem + pool kernel per workgroup: on the row
    kernel's shapes (conv rows of wo = 112 or 32 pixels) two input windows
    of 3 channels x 7 rows of 2 wo + 8 floats; otherwise two operand stages
    of the 64 x 128 tile, the stem's 256-entry tap table, a wave-boundary
    exchange row and the bias."""
    if wo in (112, 32):
        return 4 * 2 * 3 * 7 * (2 * wo + 8)
    return 4 * (2 * (64 * 32 + 128 * 32) + 2 * 256 + 4 * 2 * 32 + 64)


def _stream_conv_pool(g: Graph, lds_budget: int) -> int:
    """The packed RGB 7x7 stem conv + relu (FusedConvRelu on [Co][Kp] rows)
    whose output only feeds a 3x3 / stride 2 / pad 1 MaxPool becomes one
    FusedConvMaxPool node (inputs: x, w, bias or ""; the conv's attrs),
    lowered to nnc_hip_conv_maxpool: each workgroup pools the conv rows it
    computes. Needs Co <= 64, even conv output sizes, rows of at most 128
    pixels, N x Ho >= CONV_POOL_MIN_ROWS (unless forced with 1: the row
    kernel's shapes, 224x224 or 64x64 input)."""
    if CONV_POOL_MIN_ROWS is None:
        return 0
    fused = 0
    for conv in list(g.nodes):
        if conv.op_type != "FusedConvRelu" or len(conv.inputs) < 2:
            continue
        w = g.tensors[conv.inputs[1]]
        x = g.tensors[conv.inputs[0]]
        mid = conv.outputs[0]
        if len(w.shape) != 2 or len(x.shape) != 4 or x.shape[1] != 3 or mid in g.outputs:
            continue
        if list(conv.attrs.get("kernel_shape", [])) != [7, 7] or w.shape[0] > 64:
            continue
        users = g.consumers(mid)
        if len(users) != 1 or users[0].op_type != "MaxPool":
            continue
        pool = users[0]
        if (list(pool.attrs.get("kernel_shape", [])) != [3, 3] or list(pool.attrs.get("strides", [])) != [2, 2]
                or list(pool.attrs.get("pads", [0, 0, 0, 0])) != [1, 1, 1, 1]):
            continue
        _, _, ho, wo = g.tensors[mid].shape
        if ho % 2 or wo % 2 or wo > 128 or conv_pool_lds_bytes(wo) > lds_budget:
            continue
        if CONV_POOL_MIN_ROWS > 1:
            row_kernel = (wo in (112, 32) and x.shape[2] == 2 * ho and x.shape[3] == 2 * wo
                          and list(conv.attrs.get("strides", [])) == [2, 2])
            if not row_kernel or x.shape[0] * ho < CONV_POOL_MIN_ROWS:
                continue
        conv.op_type = "FusedConvMaxPool"
        conv.outputs = list(pool.outputs)
        conv.metadata["fused_from"] = conv.metadata.get("fused_from", [conv.name]) + [pool.name]
        conv.metadata["tile_stream"] = {"intermediate": mid, "lds_bytes": conv_pool_lds_bytes(wo),
                                        "budget": lds_budget, "hbm_bytes_saved": 2 * g.tensors[mid].nbytes}
        g.nodes.remove(pool)
        g.tensors.pop(mid, None)
        fused += 1
    return fused


def stream_tiles(g: Graph, lds_budget: int = LDS_BUDGET) -> int:
    """Stem conv + relu -> MaxPool as FusedConvMaxPool (_stream_conv_pool),
    and GlobalAveragePool -> Flatten -> Gemm (transB = 1, constant w [O, C])
    whose pooled and flattened tensors have no other reader becomes one
    FusedGapGemm node (inputs: x, w, bias or ""; the Gemm's alpha/beta),
    lowered to nnc_hip_gap_gemm_nt: each workgroup averages its images'
    planes into LDS and feeds them straight to the dot products, so the
    [N, C] pooled tensor is never written. Taken when the workgroup's
    intermediate (an image's C means, its w blocks and partial sums) fits
    `lds_budget`, at batches up to GAP_GEMM_MAX_BATCH. The decision and its
    footprint are recorded in the node's metadata["tile_stream"]."""
    fused = _stream_conv_pool(g, lds_budget)
    for gap in list(g.nodes):
        if gap.op_type != "GlobalAveragePool" or len(gap.inputs) != 1:
            continue
        x, pooled = gap.inputs[0], gap.outputs[0]
        xs = g.tensors[x].shape
        if len(xs) != 4 or pooled in g.outputs or g.tensors[x].dtype != "float32" or xs[0] > GAP_GEMM_MAX_BATCH:
            continue
        if xs[1] % 4 or xs[1] > 1024:
            continue
        users = g.consumers(pooled)
        if len(users) != 1 or users[0].op_type != "Flatten" or int(users[0].attrs.get("axis", 1)) != 1:
            continue
        flat = users[0]
        flat_out = flat.outputs[0]
        gemms = g.consumers(flat_out)
        if flat_out in g.outputs or len(gemms) != 1 or gemms[0].op_type != "Gemm":
            continue
        gm = gemms[0]
        if gm.inputs[0] != flat_out or int(gm.attrs.get("transA", 0)) != 0 or int(gm.attrs.get("transB", 0)) != 1:
            continue
        w = g.tensors[gm.inputs[1]]
        if not w.is_constant or len(w.shape) != 2 or w.shape[1] != xs[1]:
            continue
        need = gap_gemm_lds_bytes(int(xs[1]), int(xs[2]) * int(xs[3]))
        if need > lds_budget:
            continue
        bias = gm.inputs[2] if len(gm.inputs) > 2 else ""
        if bias and g.tensors[bias].numel not in (int(w.shape[0]), int(xs[0]) * int(w.shape[0])):
            continue
        gap.op_type = "FusedGapGemm"
        gap.inputs = [x, gm.inputs[1], bias]
        gap.outputs = list(gm.outputs)
        gap.attrs = {"alpha": float(gm.attrs.get("alpha", 1.0)), "beta": float(gm.attrs.get("beta", 1.0))}
        gap.metadata["fused_from"] = [gap.name, flat.name, gm.name]
        gap.metadata["tile_stream"] = {"intermediate": pooled, "lds_bytes": need, "budget": lds_budget,
                                       "hbm_bytes_saved": 2 * g.tensors[pooled].nbytes}
        g.nodes.remove(flat)
        g.nodes.remove(gm)
        g.tensors.pop(pooled, None)
        g.tensors.pop(flat_out, None)
        fused += 1
    return fused


# ---------------------------------------------------------------------------
# element-wise chains and Concat -> Split round trips (O3, mi355x target)
# ---------------------------------------------------------------------------
# Element-wise ops the chain kernel (nnc_hip_fused_eltwise) takes: step op
# (include/nnc_hip.h NNC_EW_*) and number of data operands.
EW_STEPS = {"Add": ("ADD", 2), "Sub": ("SUB", 2), "Mul": ("MUL", 2), "Div": ("DIV", 2),
            "FusedAddRelu": ("ADD_RELU", 2), "FusedAddSigmoid": ("ADD_SIGMOID", 2),
            "Relu": ("RELU", 1), "Sigmoid": ("SIGMOID", 1), "Tanh": ("TANH", 1), "Clip": ("CLIP", 1)}
EW_MAX_INPUTS, EW_MAX_STEPS = 4, 8


def _ew_node_ok(g: Graph, node: Node) -> bool:
    """A float32 element-wise node whose data operands all have its output's
    element count (the chain kernel does not broadcast)."""
    if node.op_type not in EW_STEPS or len(node.outputs) != 1:
        return False
    arity = EW_STEPS[node.op_type][1]
    out = g.tensors[node.outputs[0]]
    if out.dtype != "float32" or len(node.inputs) < arity:
        return False
    return all(node.inputs[k] and g.tensors[node.inputs[k]].dtype == "float32"
               and g.tensors[node.inputs[k]].numel == out.numel for k in range(arity))


def fuse_eltwise_chains(g: Graph) -> int:
    """Element-wise nodes each feeding only the next (an output with one
    reader, not a graph output) become one FusedEltwise node, lowered to
    nnc_hip_fused_eltwise: the chain runs in registers, its intermediates
    never reach HBM. A chain takes at most EW_MAX_STEPS nodes and
    EW_MAX_INPUTS distinct external inputs; its nodes keep their order and
    arithmetic (steps: op, x, y, lo, hi with operand -1 the running value),
    so the values are those of the op-by-op calls."""
    from .lower import clip_bounds
    from ..abi import EW_OPS
    fused = 0
    done: set[str] = set()
    for head in g.topological_sort():
        if head.name in done or not _ew_node_ok(g, head):
            continue
        chain, inputs, steps, prev = [], [], [], None
        node = head
        while True:
            op, arity = EW_STEPS[node.op_type]
            new_in = [t for t in node.inputs[:arity] if t != prev and t not in inputs]
            if len(chain) == EW_MAX_STEPS or len(inputs) + len(set(new_in)) > EW_MAX_INPUTS:
                break
            for t in new_in:
                if t not in inputs:
                    inputs.append(t)
            ops = [-1 if t == prev else inputs.index(t) for t in node.inputs[:arity]]
            lo, hi = clip_bounds(g, node) if node.op_type == "Clip" else (0.0, 0.0)
            steps.append((EW_OPS[op], ops[0], ops[1] if arity == 2 else ops[0], lo, hi))
            chain.append(node)
            prev = node.outputs[0]
            users = g.consumers(prev)
            if prev in g.outputs or len(users) != 1 or not _ew_node_ok(g, users[0]):
                break
            nxt = users[0]
            if nxt.name in done or prev not in nxt.inputs[:EW_STEPS[nxt.op_type][1]]:
                break
            node = nxt
        if len(chain) < 2:
            continue
        last = chain[-1]
        fusedn = Node(name=head.name, op_type="FusedEltwise", inputs=list(inputs), outputs=list(last.outputs),
                      attrs={"steps": [list(s) for s in steps]})
        fusedn.metadata["fused_from"] = [n.name for n in chain]
        inter = [n.outputs[0] for n in chain[:-1]]
        fusedn.metadata["tile_stream"] = {"intermediates": inter,
                                          "hbm_bytes_saved": 2 * sum(g.tensors[t].nbytes for t in inter)}
        # (in place of the last node: every external input exists by then)
        at = g.nodes.index(last)
        g.nodes[at] = fusedn
        for n in chain[:-1]:
            g.nodes.remove(n)
        done.update(n.name for n in chain)
        for t in inter:
            g.tensors.pop(t, None)
        fused += 1
    return fused


def fuse_add_layernorm(g: Graph) -> int:
    """An Add of two same-size float32 tensors whose output only a
    LayerNormalization reads (as its input, no graph output) becomes one
    FusedAddLayerNorm node (inputs: a, b, scale, bias; the LayerNorm's
    attrs), lowered to nnc_hip_add_layernorm: the sum stays in registers.
    The same bits as the Add and the LayerNorm run one after the other."""
    fused = 0
    for add in list(g.nodes):
        if add.op_type != "Add" or len(add.inputs) != 2 or add.outputs[0] in g.outputs:
            continue
        s = add.outputs[0]
        t = g.tensors[s]
        if t.dtype != "float32" or any(g.tensors[i].dtype != "float32" or g.tensors[i].numel != t.numel
                                       for i in add.inputs):
            continue
        users = g.consumers(s)
        if len(users) != 1 or users[0].op_type != "LayerNormalization" or users[0].inputs[0] != s:
            continue
        ln = users[0]
        ln.op_type = "FusedAddLayerNorm"
        ln.inputs = list(add.inputs) + list(ln.inputs[1:3]) + [""] * (3 - len(ln.inputs))
        ln.metadata["fused_from"] = [add.name, ln.name]
        ln.metadata["tile_stream"] = {"intermediate": s, "hbm_bytes_saved": 2 * t.nbytes}
        g.nodes.remove(add)
        g.tensors.pop(s, None)
        fused += 1
    return fused


def fuse_scaled_softmax(g: Graph) -> int:
    """A Div of a float32 tensor by a one-element float32 tensor whose
    output only a Softmax reads (no graph output) becomes one ScaledSoftmax
    node (inputs: x, divisor; the Softmax's attrs), lowered to
    nnc_hip_scaled_softmax: attention's score scaling applied as the rows
    are loaded. The same bits as the Div and the Softmax one after the
    other."""
    fused = 0
    for div in list(g.nodes):
        if div.op_type != "Div" or len(div.inputs) != 2 or div.outputs[0] in g.outputs:
            continue
        q = div.outputs[0]
        x, d = (g.tensors[i] for i in div.inputs)
        t = g.tensors[q]
        if any(v.dtype != "float32" for v in (x, d, t)) or d.numel != 1 or x.numel != t.numel:
            continue
        users = g.consumers(q)
        if len(users) != 1 or users[0].op_type != "Softmax" or users[0].inputs[0] != q:
            continue
        sm = users[0]
        sm.op_type = "ScaledSoftmax"
        sm.inputs = list(div.inputs)
        sm.metadata["fused_from"] = [div.name, sm.name]
        sm.metadata["tile_stream"] = {"intermediate": q, "hbm_bytes_saved": 2 * t.nbytes}
        g.nodes.remove(div)
        g.tensors.pop(q, None)
        fused += 1
    return fused


def fuse_split_transposes(g: Graph) -> int:
    """A float32 Split along the last axis whose every piece is read only by
    a Reshape, itself read only by a Transpose (attention's head split of
    the fused QKV projection), loses the Split and the Reshapes: each
    Transpose becomes a SliceTranspose of the unsplit tensor (attrs perm,
    col0, width), lowered to nnc_hip_transpose_slice. A copy of the same
    elements: the bits of the Split, the Reshape and the Transpose."""
    fused = 0
    for split in list(g.nodes):
        if split.op_type != "Split" or not split.inputs or not split.outputs:
            continue
        x = g.tensors[split.inputs[0]]
        nd = len(x.shape)
        if nd < 1 or x.dtype != "float32" or int(split.attrs.get("axis", 0)) % nd != nd - 1:
            continue
        chains = []
        for piece in split.outputs:
            users = g.consumers(piece)
            if piece in g.outputs or len(users) != 1 or users[0].op_type != "Reshape" or users[0].inputs[0] != piece:
                break
            rs = users[0]
            tr = g.consumers(rs.outputs[0])
            if rs.outputs[0] in g.outputs or len(tr) != 1 or tr[0].op_type != "Transpose" or tr[0].inputs[0] != rs.outputs[0]:
                break
            chains.append((piece, rs, tr[0]))
        if len(chains) != len(split.outputs):
            continue
        widths = [int(g.tensors[p].shape[-1]) for p, _, _ in chains]
        if sum(widths) != int(x.shape[-1]) or x.shape[-1] >= 1 << 31:
            continue
        col0 = 0
        for (piece, rs, tr), w in zip(chains, widths):
            vnd = len(g.tensors[rs.outputs[0]].shape)
            tr.attrs["perm"] = [int(v) for v in (tr.attrs.get("perm") or range(vnd - 1, -1, -1))]
            tr.op_type = "SliceTranspose"
            tr.inputs = [split.inputs[0]]
            tr.attrs["col0"], tr.attrs["width"] = col0, w
            tr.metadata["fused_from"] = [split.name, rs.name, tr.name]
            col0 += w
            g.nodes.remove(rs)
            for t in rs.outputs + [piece]:
                g.tensors.pop(t, None)
            for c in rs.inputs[1:]:
                if c in g.tensors and not g.consumers(c) and c not in g.outputs:
                    g.tensors.pop(c, None)
        g.nodes.remove(split)
        fused += 1
    return fused


ATTENTION_HEAD_DIMS = (32, 64)
ATTENTION_MAX_SEQ = 128


def _only_reader(g: Graph, tensor: str, op_type: str, index: int | None = 0):
    """The one node reading `tensor` (no graph output), if it is an
    `op_type` reading it at input `index` (any input if None)."""
    if tensor in g.outputs:
        return None
    users = g.consumers(tensor)
    if len(users) != 1 or users[0].op_type != op_type:
        return None
    if index is not None and (len(users[0].inputs) <= index or users[0].inputs[index] != tensor):
        return None
    return users[0]


def fuse_attention(g: Graph) -> int:
    """A transformer layer's attention block - after fuse_split_transposes,
    compose_transposes and fuse_scaled_softmax: SliceTranspose Q (perm
    0,2,1,3) and K^T (perm 0,2,3,1) of one QKV tensor into a MatMul, a
    ScaledSoftmax of its scores over the last axis, a MatMul with
    SliceTranspose V (perm 0,2,1,3), and the head merge Transpose (perm
    0,2,1,3), each intermediate read only by the next node - becomes one
    Attention node (inputs: the QKV tensor, the divisor; attrs batch, seq,
    heads, head_dim, q_col, k_col, v_col), lowered to nnc_hip_attention.
    Taken for float32, head_dim in ATTENTION_HEAD_DIMS, seq a multiple of 32
    up to ATTENTION_MAX_SEQ, QKV rows and column offsets multiples of four
    floats; the intermediates (scores, probabilities, per-head Q, K^T, V and
    context) never reach HBM."""
    fused = 0
    for mm1 in list(g.nodes):
        if mm1.op_type != "MatMul" or len(mm1.inputs) != 2:
            continue
        tq, tk = (g.producer(i) for i in mm1.inputs)
        if tq is None or tk is None or tq.op_type != "SliceTranspose" or tk.op_type != "SliceTranspose":
            continue
        if tq.inputs[0] != tk.inputs[0] or [int(v) for v in tq.attrs["perm"]] != [0, 2, 1, 3] or \
                [int(v) for v in tk.attrs["perm"]] != [0, 2, 3, 1]:
            continue
        if _only_reader(g, tq.outputs[0], "MatMul", 0) is not mm1 or _only_reader(g, tk.outputs[0], "MatMul", 1) is not mm1:
            continue
        sm = _only_reader(g, mm1.outputs[0], "ScaledSoftmax")
        if sm is None or int(sm.attrs.get("axis", -1)) not in (-1, 3):
            continue
        mm2 = _only_reader(g, sm.outputs[0], "MatMul", 0)
        if mm2 is None:
            continue
        tv = g.producer(mm2.inputs[1])
        if tv is None or tv.op_type != "SliceTranspose" or tv.inputs[0] != tq.inputs[0] or \
                [int(v) for v in tv.attrs["perm"]] != [0, 2, 1, 3] or \
                _only_reader(g, tv.outputs[0], "MatMul", 1) is not mm2:
            continue
        tr = _only_reader(g, mm2.outputs[0], "Transpose")
        if tr is None or [int(v) for v in (tr.attrs.get("perm") or [])] != [0, 2, 1, 3]:
            continue
        qkv = g.tensors[tq.inputs[0]]
        qt = g.tensors[tq.outputs[0]]
        if len(qt.shape) != 4 or any(g.tensors[t].dtype != "float32"
                                     for t in (tq.inputs[0], sm.inputs[1], tr.outputs[0])):
            continue
        batch, heads, seq, dh = (int(v) for v in qt.shape)
        width = int(qkv.shape[-1])
        if g.tensors[sm.inputs[1]].numel != 1 or qkv.numel != batch * seq * width:
            continue
        if dh not in ATTENTION_HEAD_DIMS or seq % 32 or seq > ATTENTION_MAX_SEQ or width % 4:
            continue
        cols = [int(t.attrs["col0"]) for t in (tq, tk, tv)]
        if any(c % 4 or int(t.attrs["width"]) != heads * dh for c, t in zip(cols, (tq, tk, tv))):
            continue
        if list(g.tensors[tk.outputs[0]].shape) != [batch, heads, dh, seq] or \
                list(g.tensors[tv.outputs[0]].shape) != [batch, heads, seq, dh]:
            continue
        dead = [tq, tk, tv, mm1, sm, mm2]
        mids = [tq.outputs[0], tk.outputs[0], tv.outputs[0], mm1.outputs[0], sm.outputs[0], mm2.outputs[0]]
        tr.op_type = "Attention"
        tr.inputs = [tq.inputs[0], sm.inputs[1]]
        tr.attrs = {"batch": batch, "seq": seq, "heads": heads, "head_dim": dh,
                    "q_col": cols[0], "k_col": cols[1], "v_col": cols[2]}
        tr.metadata["fused_from"] = [n.name for n in dead] + [tr.name]
        tr.metadata["tile_stream"] = {"intermediate": mids,
                                      "hbm_bytes_saved": 2 * sum(g.tensors[t].nbytes for t in mids)}
        for n in dead:
            g.nodes.remove(n)
        for t in mids:
            g.tensors.pop(t, None)
        fused += 1
    return fused


def compose_transposes(g: Graph) -> int:
    """A Transpose whose input is another Transpose's output read by nothing
    else (and no graph output) becomes one Transpose of the first's input
    with the composed permutation: out.shape[i] = x.shape[p1[p2[i]]], the
    same element moves, one copy instead of two."""
    merged = 0
    for t2 in list(g.nodes):
        if t2.op_type != "Transpose" or not t2.inputs:
            continue
        t1 = g.producer(t2.inputs[0])
        if t1 is None or t1.op_type != "Transpose" or t1.outputs[0] in g.outputs:
            continue
        if len(g.consumers(t1.outputs[0])) != 1:
            continue
        nd = len(g.tensors[t1.inputs[0]].shape)
        p1 = list(t1.attrs.get("perm") or range(nd - 1, -1, -1))
        p2 = list(t2.attrs.get("perm") or range(nd - 1, -1, -1))
        if len(p1) != nd or len(p2) != nd:
            continue
        mid = t1.outputs[0]
        t2.inputs = [t1.inputs[0]] + list(t2.inputs[1:])
        t2.attrs = {**t2.attrs, "perm": [int(p1[p2[i]]) for i in range(nd)]}
        t2.metadata["fused_from"] = [t1.name, t2.name]
        g.nodes.remove(t1)
        g.tensors.pop(mid, None)
        merged += 1
    return merged


def eliminate_concat_split(g: Graph) -> int:
    """A Split whose input is a Concat along the same axis into the same
    pieces (the Concat's output read by nothing else, neither result a graph
    output) hands the Concat's inputs straight to the Split's readers: both
    copies disappear and every value is unchanged."""
    removed = 0
    for split in list(g.nodes):
        if split.op_type != "Split" or not split.inputs:
            continue
        cat = g.producer(split.inputs[0])
        if cat is None or cat.op_type != "Concat" or cat.outputs[0] in g.outputs:
            continue
        if len(g.consumers(cat.outputs[0])) != 1 or any(o in g.outputs for o in split.outputs):
            continue
        nd = len(g.tensors[cat.outputs[0]].shape)
        ax_c, ax_s = int(cat.attrs.get("axis", 0)) % nd, int(split.attrs.get("axis", 0)) % nd
        if ax_c != ax_s or len(cat.inputs) != len(split.outputs):
            continue
        if any(list(g.tensors[a].shape) != list(g.tensors[b].shape) or g.tensors[a].dtype != g.tensors[b].dtype
               for a, b in zip(cat.inputs, split.outputs)):
            continue
        rename = dict(zip(split.outputs, cat.inputs))
        for c in g.nodes:
            c.inputs = [rename.get(i, i) for i in c.inputs]
        g.nodes.remove(split)
        g.nodes.remove(cat)
        for t in list(split.outputs) + [cat.outputs[0]]:
            g.tensors.pop(t, None)
        removed += 1
    return removed


# ---------------------------------------------------------------------------
# liveness and the arena plan
# ---------------------------------------------------------------------------
@dataclass
class Liveness:
    start: int
    end: int
    is_input: bool = False
    is_output: bool = False


def liveness(g: Graph, order: list[Node], concurrent: list[list[str]] | None = None) -> dict[str, Liveness]:
    """[first definition, last use] per non-constant tensor over `order`
    (passes/liveness.py:23-132). Graph inputs are live from step 0, graph
    outputs to the end. Every tensor a node of a `concurrent` group reads or
    writes stays live to the group's last step, so nothing one member touches
    is freed (and reused, or written in place) while another may still run."""
    live: dict[str, Liveness] = {}
    last = len(order)
    for name in g.inputs:
        live[name] = Liveness(0, 0, is_input=True)
    for idx, node in enumerate(order):
        for o in node.outputs:
            if o and not g.tensors[o].is_constant and g.tensors[o].pool == "fast":
                live.setdefault(o, Liveness(idx, idx))
        for i in node.inputs:
            if i in live:
                live[i].end = max(live[i].end, idx)
    for name in g.outputs:
        if name in live:
            live[name].end = last
            live[name].is_output = True
    for name in g.inputs:  # inputs stay resident across repeated runs
        live[name].end = last
    pos = {n.name: i for i, n in enumerate(order)}
    for group in concurrent or []:
        members = [order[pos[n]] for n in group if n in pos]
        if not members:
            continue
        end = max(pos[n.name] for n in members)
        for n in members:
            for t in list(n.inputs) + list(n.outputs):
                if t in live:
                    live[t].end = max(live[t].end, end)
    return live


@dataclass
class MemoryPlan:
    """Offsets of every tensor in one arena: [activations | constants]."""
    offsets: dict[str, int] = field(default_factory=dict)
    activation_bytes: int = 0
    constant_offset: int = 0
    total_bytes: int = 0
    inplace: dict[str, str] = field(default_factory=dict)  # output -> reused input
    aliases: dict[str, str] = field(default_factory=dict)  # view output -> its input (no copy)
    # spilled copies: offsets in the spill pool (pinned host memory)
    slow_offsets: dict[str, int] = field(default_factory=dict)
    slow_bytes: int = 0
    first_over: int | None = None  # first node whose allocation passed the budget


def _align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


# ops whose output is the input's bytes under another shape
VIEW_OPS = {"Flatten", "Reshape", "Squeeze", "Unsqueeze", "Identity"}


def plan_memory(g: Graph, order: list[Node], strategy: str = "cost_aware",
                max_memory: int | None = None, alias_views: bool = False,
                concurrent: list[list[str]] | None = None, budget: int | None = None) -> MemoryPlan:
    """Greedy offset assignment over the execution order.

    alias_views (mi355x O3): a view op whose input dies there gets the
    input's offset and no call at all (plan.aliases).

    basic:       every activation gets its own region (no reuse).
    cost_aware:  freed regions are reused best-fit; element-wise nodes write
                 over a same-sized input that dies there.
    Raises ValueError when the activations exceed max_memory (fit_memory
    spills instead). With `budget`, plan.first_over is the first node at
    which the arena grew past it. Spilled copies (pool "slow") get offsets
    in the spill pool, one region each."""
    live = liveness(g, order, concurrent)
    sizes = {n: _align(g.tensors[n].nbytes) for n in live}
    plan = MemoryPlan()
    free: list[tuple[int, int]] = []  # (offset, size)
    top = 0
    at = 0  # node being planned

    def take(size: int) -> int:
        off = _take(size)
        if budget is not None and plan.first_over is None and off + size > budget:
            plan.first_over = at
        return off

    def _take(size: int) -> int:
        nonlocal top
        if strategy == "cost_aware":
            best = None
            for k, (off, sz) in enumerate(free):
                if sz >= size and (best is None or sz < free[best][1]):
                    best = k
            if best is not None:
                off, sz = free.pop(best)
                if sz > size:
                    free.append((off + size, sz - size))
                return off
        off = top
        top += size
        return off

    def release(off: int, size: int) -> None:
        if strategy != "cost_aware":
            return
        free.append((off, size))
        free.sort()
        merged = []
        for o, s in free:
            if merged and merged[-1][0] + merged[-1][1] == o:
                merged[-1] = (merged[-1][0], merged[-1][1] + s)
            else:
                merged.append((o, s))
        free[:] = merged
        # a free block ending at the top shrinks the pool
        nonlocal top
        if free and free[-1][0] + free[-1][1] == top:
            top = free.pop()[0]

    for name in g.inputs:
        plan.offsets[name] = take(sizes[name])
    for idx, node in enumerate(order):
        at = idx
        reused = set()
        for o in node.outputs:
            if not o or o not in live or o in plan.offsets:
                continue
            slot = None
            if strategy == "cost_aware" and alias_views and node.op_type in VIEW_OPS and node.inputs:
                i = node.inputs[0]
                li = live.get(i)
                if (li and li.end == idx and not li.is_output and not li.is_input and i in plan.offsets
                        and i not in reused and sizes[i] == sizes[o]
                        and g.tensors[i].nbytes == g.tensors[o].nbytes):
                    slot = plan.offsets[i]
                    reused.add(i)
                    plan.inplace[o] = i
                    plan.aliases[o] = i
            if slot is None and strategy == "cost_aware" and node.op_type in INPLACE_OPS:
                allowed = INPLACE_INPUTS.get(node.op_type)
                for k, i in enumerate(node.inputs):
                    if allowed is not None and k not in allowed:
                        continue
                    # a tensor the node also reads through a restricted input
                    # (the fused conv's image, relu(conv(h) + h)) is still read
                    # by other workgroups while finished tiles are stored
                    if allowed is not None and any(j == i for kk, j in enumerate(node.inputs)
                                                   if kk not in allowed):
                        continue
                    li = live.get(i)
                    if (li and li.end == idx and not li.is_output and not li.is_input
                            and i in plan.offsets and i not in reused and sizes[i] == sizes[o]):
                        slot = plan.offsets[i]
                        reused.add(i)
                        plan.inplace[o] = i
                        break
            plan.offsets[o] = slot if slot is not None else take(sizes[o])
        # graph inputs stay resident so nnc_run() can be repeated on them
        for i in set(node.inputs):
            li = live.get(i)
            if li and li.end == idx and not li.is_output and not li.is_input and i not in reused:
                release(plan.offsets[i], sizes[i])
        # outputs nobody reads die immediately
        for o in node.outputs:
            lo = live.get(o)
            if lo and lo.end == idx and not lo.is_output and o not in node.inputs:
                release(plan.offsets[o], sizes[o])
    plan.activation_bytes = _align(max([top] + [plan.offsets[n] + sizes[n] for n in plan.offsets]))
    if max_memory is not None and plan.activation_bytes > max_memory:
        raise ValueError(f"max_memory ({max_memory}) < peak activation footprint "
                         f"({plan.activation_bytes}) of the arena plan")
    off = plan.activation_bytes
    plan.constant_offset = off
    for name, t in g.constants.items():
        plan.offsets[name] = off
        off += _align(t.nbytes)
    plan.total_bytes = _align(off)
    slow = 0
    for node in order:
        for o in node.outputs:
            if o and g.tensors[o].pool == "slow" and o not in plan.slow_offsets:
                plan.slow_offsets[o] = slow
                slow += _align(g.tensors[o].nbytes)
    plan.slow_bytes = slow
    return plan


def check_plan(g: Graph, order: list[Node], plan: MemoryPlan, concurrent: list[list[str]] | None = None) -> None:
    """Invariants: simultaneously live tensors never overlap (except an
    in-place output and the input it replaces), every offset aligned, every
    tensor inside the arena."""
    live = liveness(g, order, concurrent)
    names = list(live)
    for n, off in plan.slow_offsets.items():
        assert off % ALIGN == 0 and off + g.tensors[n].nbytes <= plan.slow_bytes, n
    for n in plan.offsets:
        assert plan.offsets[n] % ALIGN == 0, n
        assert plan.offsets[n] + g.tensors[n].nbytes <= plan.total_bytes, n
    for a_i, a in enumerate(names):
        la, oa, sa = live[a], plan.offsets[a], g.tensors[a].nbytes
        for b in names[a_i + 1:]:
            lb, ob, sb = live[b], plan.offsets[b], g.tensors[b].nbytes
            overlap_t = la.start <= lb.end and lb.start <= la.end
            overlap_m = oa < ob + sb and ob < oa + sa
            if overlap_t and overlap_m:
                pair = plan.inplace.get(a) == b or plan.inplace.get(b) == a
                if not pair:
                    raise AssertionError(f"{a} and {b} overlap in time and memory")


# ---------------------------------------------------------------------------
# a fast-memory budget: spill to pinned host memory, reload before next use
# ---------------------------------------------------------------------------
SPILL_OPS = ("Spill", "Reload")


def _fresh(names, base: str) -> str:
    k, name = 0, base
    while name in names:
        k += 1
        name = f"{base}{k}"
    return name


def _spill_victim(g: Graph, order: list[Node], idx: int, need: int) -> str | None:
    """The tensor to spill when the arena passes its budget at node `idx`:
    live across the node (made before it, read after it) and not read by
    it; graph inputs and outputs stay resident. Prefer one that alone frees
    what is missing, then the one read again last (Belady's rule), then the
    larger."""
    live = liveness(g, order)
    reads = set(order[idx].inputs)
    best, best_key = None, None
    for t, lv in live.items():
        if lv.is_input or lv.is_output or t in reads or not (lv.start < idx < lv.end):
            continue
        nxt = next(k for k in range(idx + 1, len(order)) if t in order[k].inputs)
        size = g.tensors[t].nbytes
        key = (_align(size) >= need, nxt, size)
        if best_key is None or key > best_key:
            best, best_key = t, key
    return best


def _insert_spill(g: Graph, order: list[Node], t: str, idx: int) -> list[Node]:
    """Spill `t` after its last read before node `idx` (or after its
    producer), reload it into a new tensor before its next read after
    `idx`; later nodes read the reloaded tensor."""
    reads = [k for k, n in enumerate(order) if t in n.inputs]
    made = next(k for k, n in enumerate(order) if t in n.outputs)
    after = max([k for k in reads if k < idx] + [made])
    nxt = min(k for k in reads if k > idx)
    info = g.tensors[t]
    held = _fresh(g.tensors, f"{t}.spilled")
    g.add_tensor(TensorInfo(held, info.shape, info.dtype, pool="slow"))
    back = _fresh(g.tensors, f"{t}.reloaded")
    g.add_tensor(TensorInfo(back, info.shape, info.dtype))
    names = {n.name for n in order}
    spill = Node(_fresh(names, f"spill_{t}"), "Spill", [t], [held])
    names.add(spill.name)
    reload = Node(_fresh(names, f"reload_{t}"), "Reload", [held], [back])
    for n in order[nxt:]:
        n.inputs = [back if i == t else i for i in n.inputs]
    new = order[:after + 1] + [spill] + order[after + 1:nxt] + [reload] + order[nxt:]
    g.nodes = list(new)
    return new


def fit_memory(g: Graph, order: list[Node], max_memory: int, plan_fn) -> tuple[list[Node], MemoryPlan]:
    """Meet a fast-memory budget (the HBM arena's activation region) by
    spilling. `plan_fn(order, budget)` plans an order; while the plan passes
    `max_memory`, the tensor chosen by _spill_victim at the first node
    where the arena grew past the budget is spilled to the spill pool
    (pinned host memory) and reloaded before its next read, and the order is
    planned again. Same contract as the reference's cost_aware allocator
    with a budget (cost_aware_allocator.py:63-102, 267-377; spill and
    reload copies, model_source.py:259-290): the fast pool stays within
    max_memory, and a budget that cannot hold what one node needs at once
    raises ValueError. The eviction rule is this module's own."""
    for _ in range(8 * len(order) + 64):
        plan = plan_fn(order, max_memory)
        if plan.activation_bytes <= max_memory:
            return order, plan
        idx = plan.first_over if plan.first_over is not None else len(order) - 1
        victim = _spill_victim(g, order, idx, plan.activation_bytes - max_memory)
        if victim is None:
            node = order[idx].name if order else "(graph inputs)"
            raise ValueError(f"max_memory ({max_memory}) < the fast memory node {node} needs with every "
                             f"tensor it cannot spill resident (plan peak {plan.activation_bytes})")
        order = _insert_spill(g, order, victim, idx)
    raise ValueError(f"max_memory ({max_memory}): spilling did not converge")


# ---------------------------------------------------------------------------
# independent branches on the second library stream (mi355x O3)
# ---------------------------------------------------------------------------


def conv_flops(g: Graph, node: Node) -> float:
    """2 * Co * (N * Ho * Wo) * (Ci * kh * kw) of a convolution node (weights
    [Co][Ci][kh][kw] or tap-major packed; the output shape gives N*Ho*Wo)."""
    w = g.tensors[node.inputs[1]]
    out = g.tensors[node.outputs[0]].shape
    k = 1
    for d in w.shape[1:]:
        k *= int(d)
    return 2.0 * int(w.shape[0]) * (int(out[0]) * int(out[2]) * int(out[3])) * k


@dataclass
class Branch:
    """`side` runs on stream 1 from the fork until the join before `join`;
    `main` are the nodes stream 0 runs meanwhile (between the fork and the
    join in execution order)."""
    side: str
    main: list[str]
    join: str


def find_branches(g: Graph, order: list[Node], max_flops: float) -> list[Branch]:
    """Side branches for the second stream: a convolution D whose only
    activation input X has exactly one other consumer A, and whose output
    has exactly one consumer J - ResNet's 1x1 downsample next to the
    block's first 3x3 convolution, joined by the residual add (either of
    the two can be D). The main branch is every node from A (or D, if
    earlier) up to J; taken only while D and the main branch's convolutions
    each stay within `max_flops` (two concurrent kernels pay off while
    neither fills the GPU)."""
    pos = {n.name: i for i, n in enumerate(order)}
    consumers: dict[str, list[Node]] = {}
    for n in order:
        for t in n.inputs:
            consumers.setdefault(t, []).append(n)
    taken: set[str] = set()
    out: list[Branch] = []
    for d in order:
        if d.op_type not in CONV_OPS or d.name in taken:
            continue
        acts = [t for t in d.inputs if t and t in g.tensors and not g.tensors[t].is_constant]
        if len(acts) != 1 or len(d.outputs) != 1:
            continue
        others = [c for c in consumers.get(acts[0], []) if c.name != d.name]
        readers = consumers.get(d.outputs[0], [])
        if len(others) != 1 or len(readers) != 1 or d.outputs[0] in g.outputs:
            continue
        a, j = others[0], readers[0]
        lo, hi = min(pos[a.name], pos[d.name]), pos[j.name]
        if pos[a.name] >= hi or pos[d.name] >= hi:
            continue
        main = [order[i] for i in range(lo, hi) if order[i].name != d.name]
        if not main or any(n.name in taken for n in main + [j]):
            continue
        # the join must read what the main branch produced
        made = {t for n in main for t in n.outputs}
        if not any(t in made for t in j.inputs):
            continue
        flops = sum(conv_flops(g, n) for n in main if n.op_type in FLOP_CONV_OPS)
        if max(flops, conv_flops(g, d)) > max_flops:
            continue
        out.append(Branch(d.name, [n.name for n in main], j.name))
        taken.update([d.name, j.name] + [n.name for n in main])
    return out


def branch_calls(calls: list, branches: list[Branch], make_call) -> list:
    """The call list with each branch's side call moved to a fork placed
    before the branch's first main call (or before its join, if the main
    nodes made no call), on stream 1, and a join before the join node's call.
    `make_call(op, args)` builds a call."""
    if not branches:
        return calls
    side_calls = {c.node: c for c in calls}
    main_of = {n: b for b in branches for n in b.main}
    join_of = {b.join: b for b in branches}
    side_nodes = {b.side for b in branches}
    forked: set[str] = set()

    def fork(b: Branch) -> list:
        forked.add(b.side)
        return [make_call("nnc_hip_stream_fork", []), make_call("nnc_hip_stream_select", [("i", 1)]),
                side_calls[b.side], make_call("nnc_hip_stream_select", [("i", 0)])]

    out = []
    for c in calls:
        if c.node in side_nodes:
            continue  # emitted at its fork
        b = main_of.get(c.node)
        if b is not None and b.side not in forked:
            out += fork(b)
        b = join_of.get(c.node)
        if b is not None:
            if b.side not in forked:
                out += fork(b)
            out.append(make_call("nnc_hip_stream_join", []))
        out.append(c)
    return out
