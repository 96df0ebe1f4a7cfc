"""The ONNX Runtime execution provider's partitioning without a GPU
(arthip_ep_get_capability with no device check).

Mirrors the reference's capability rules (src/onnxruntime-hip/
hip_execution_provider.cc:22-177 IsNodeSupported, 181-335 GetCapability) and
the cases its EP tests drive through ONNX Runtime (tests/correctness/
test_ep.py): the fp32-boundary conv fixture is claimed whole (P1-4), a region
with two activation inputs is not claimed (P2-17), a graph input shared by two
convs is one deduplicated input (P2-17). ONNX Runtime is not installed, so the
partition is checked directly, node by node.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from arthip_amd import onnx_proto as op
from arthip_amd.engine import EngineError, get_capability
from tests.fixtures import _conv, _half, _model, fused_node_graph, kern, linspace

GOLDEN = Path(__file__).resolve().parent / "golden"
F16, F32 = op.FLOAT16, op.FLOAT


def conv_model(*, c=4, m=4, k=3, extra=None, bias_dtype=np.float16, **conv_attrs):
    """One Conv node (weights from an initializer) with attribute overrides."""
    w = kern(21, m, c, k)
    attrs = dict(kernel_shape=[k, k], pads=[1, 1, 1, 1], strides=[1, 1], dilations=[1, 1],
                 group=1)
    attrs.update(conv_attrs)
    attrs = {a: v for a, v in attrs.items() if v is not None}
    node = op.node("Conv", ["x", "w", "b"], ["y"], **attrs)
    b = linspace(m).astype(bias_dtype)
    inits = [_half("w", w), op.tensor("b", b)]
    return _model([node] + (extra or []), "x", [1, c, "h", "w"], F16, "y", [1, m, "h", "w"], F16,
                  inits)


def claims(model):
    return get_capability(model)


# ---------------------------------------------------------------------------
# Whole-model claims and the single-input / single-output rule
# ---------------------------------------------------------------------------

def test_fp32_boundary_conv_is_claimed_whole(fixtures):
    assert claims(fixtures.get("ep_conv_fp32io").model) == [[0, 1, 2]]


def test_two_activation_inputs_are_not_claimed():
    g = op.Graph(nodes=[op.node("Add", ["x1", "x2"], ["y"])],
                 inputs=[op.value_info("x1", F16, [1, 4, "h", "w"]),
                         op.value_info("x2", F16, [1, 4, "h", "w"])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"])])
    assert claims(op.Model(graph=g)) == []


def test_shared_graph_input_is_deduplicated(fixtures):
    assert claims(fixtures.get("ep_two_convs_one_input").model) == [[0, 1, 2]]


def test_shipped_luma_model_is_claimed_whole():
    m = op.load(GOLDEN / "ArtCNN_R8F64_fp16.onnx")
    assert claims(m) == [list(range(len(m.graph.nodes)))]


def test_fp32_model_is_not_claimed_but_its_fp16_conversion_is():
    from oracle.convert import to_fp16
    m = op.load(GOLDEN / "ArtCNN_R8F64_Chroma.onnx")
    assert claims(m) == []
    conv = to_fp16(m, cast_input=True, cast_output=True)
    assert claims(conv) == [list(range(len(conv.graph.nodes)))]


def test_unsupported_node_splits_the_graph():
    w1, w2 = kern(31, 4, 4), kern(32, 4, 4)
    nodes = [_conv("x", "w1", None, "a"),
             op.node("Cast", ["a"], ["a32"], to=F32),    # not at a graph output
             op.node("Cast", ["a32"], ["a16"], to=F16),  # not from a graph input
             _conv("a16", "w2", None, "y")]
    m = _model(nodes, "x", [1, 4, "h", "w"], F16, "y", [1, 4, "h", "w"], F16,
               [_half("w1", w1), _half("w2", w2)])
    assert claims(m) == [[0], [3]]


def test_output_needed_outside_the_run_blocks_the_claim():
    w1, w2 = kern(33, 4, 4), kern(34, 4, 4)
    nodes = [_conv("x", "w1", None, "a"), _conv("a", "w2", None, "b"),
             op.node("Cast", ["b"], ["b32"], to=F32), op.node("Cast", ["b32"], ["c"], to=F16),
             op.node("Add", ["a", "c"], ["y"])]
    m = _model(nodes, "x", [1, 4, "h", "w"], F16, "y", [1, 4, "h", "w"], F16,
               [_half("w1", w1), _half("w2", w2)])
    # Run [0, 1] exports both a and b; run [4] reads two activations.
    assert claims(m) == []


def test_graph_output_consumed_inside_is_still_exported():
    w1, w2 = kern(35, 4, 4), kern(36, 4, 4)
    nodes = [_conv("x", "w1", None, "a"), _conv("a", "w2", None, "y")]
    g = op.Graph(nodes=nodes, initializers=[_half("w1", w1), _half("w2", w2)],
                 inputs=[op.value_info("x", F16, [1, 4, "h", "w"])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"]),
                          op.value_info("a", F16, [1, 4, "h", "w"])])
    assert claims(op.Model(graph=g)) == []  # two needed outputs


def test_nodes_out_of_topological_order_are_an_error():
    w1, w2 = kern(37, 4, 4), kern(38, 4, 4)
    nodes = [_conv("a", "w2", None, "y"), _conv("x", "w1", None, "a")]
    m = _model(nodes, "x", [1, 4, "h", "w"], F16, "y", [1, 4, "h", "w"], F16,
               [_half("w1", w1), _half("w2", w2)])
    with pytest.raises(EngineError, match="topological"):
        claims(m)


# ---------------------------------------------------------------------------
# IsNodeSupported, node by node
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("attrs,claimed", [
    (dict(), True),
    (dict(pads=[1, 0, 1, 0]), False),          # asymmetric: another convolution
    (dict(pads=[0, 0, 0, 0]), False),
    (dict(pads=None), False),                  # no padding at all
    (dict(pads=None, auto_pad="SAME_UPPER"), True),
    (dict(pads=None, auto_pad="SAME_LOWER"), True),
    (dict(pads=None, auto_pad="VALID"), False),
    (dict(auto_pad="NOTSET"), True),
    (dict(strides=[2, 2]), False),
    (dict(dilations=[2, 2]), False),
    (dict(group=2), False),
], ids=["plain", "pads-1010", "pads-0", "no-pads", "same-upper", "same-lower", "valid",
        "notset", "stride2", "dilation2", "group2"])
def test_conv_attributes(attrs, claimed):
    assert bool(claims(conv_model(**attrs))) == claimed


def test_conv_kernel_and_dtype_rules():
    assert claims(conv_model(k=5, kernel_shape=[5, 5], pads=[2, 2, 2, 2])) == []
    assert claims(conv_model(bias_dtype=np.float32)) == []          # fp16 tensors only
    assert claims(conv_model(c=97, m=4)) == []                      # beyond the engine's C limit
    assert claims(conv_model(c=4, m=129)) == []                     # beyond its M limit
    assert claims(conv_model(c=96, m=128)) == [[0]]


def test_weight_must_be_an_initializer():
    g = op.Graph(nodes=[op.node("Conv", ["x", "w"], ["y"], kernel_shape=[3, 3],
                                pads=[1, 1, 1, 1])],
                 inputs=[op.value_info("x", F16, [1, 4, "h", "w"]),
                         op.value_info("w", F16, [4, 4, 3, 3])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"])])
    assert claims(op.Model(graph=g)) == []


def _tail(node, inits=(), inputs=None):
    """conv -> node, the node's output the graph output."""
    w = kern(41, 4, 4)
    nodes = [_conv("x", "w", None, "a"), node]
    return _model(nodes, "x", [1, 4, "h", "w"], F16, node.outputs[0], [1, 4, "h", "w"], F16,
                  [_half("w", w)] + list(inits), inputs=inputs)


def test_depth_to_space_rules():
    assert claims(_tail(op.node("DepthToSpace", ["a"], ["y"], blocksize=2, mode="DCR"))) == [[0, 1]]
    assert claims(_tail(op.node("DepthToSpace", ["a"], ["y"], blocksize=2))) == [[0, 1]]
    assert claims(_tail(op.node("DepthToSpace", ["a"], ["y"], blocksize=2, mode="CRD"))) == [[0]]
    assert claims(_tail(op.node("DepthToSpace", ["a"], ["y"], blocksize=0))) == [[0]]


def test_clip_bounds_must_be_initializers():
    lo, hi = op.tensor("lo", np.float16(0.0)), op.tensor("hi", np.float16(1.0))
    assert claims(_tail(op.node("Clip", ["a", "lo", "hi"], ["y"]), [lo, hi])) == [[0, 1]]
    assert claims(_tail(op.node("Clip", ["a", "", "hi"], ["y"]), [hi])) == [[0, 1]]
    dyn = [op.value_info("x", F16, [1, 4, "h", "w"]), op.value_info("hi", F16, [])]
    assert claims(_tail(op.node("Clip", ["a", "lo", "hi"], ["y"]), [lo], inputs=dyn)) == [[0]]


def test_relu_and_domains():
    assert claims(_tail(op.node("Relu", ["a"], ["y"]))) == [[0, 1]]
    custom = op.node("Relu", ["a"], ["y"])
    custom.domain = "com.example"
    assert claims(_tail(custom)) == [[0]]
    assert claims(_tail(op.node("Tanh", ["a"], ["y"]))) == [[0]]


def test_boundary_casts_only():
    w = kern(42, 1, 1)
    inner = [op.node("Cast", ["x"], ["x16"], to=F16), _conv("x16", "w", None, "a"),
             op.node("Cast", ["a"], ["y"], to=F32)]
    m = _model(inner, "x", [1, 1, "h", "w"], F32, "y", [1, 1, "h", "w"], F32, [_half("w", w)])
    assert claims(m) == [[0, 1, 2]]
    # A Cast to fp16 whose input is not a graph input is not a boundary Cast.
    w2 = kern(43, 1, 1)
    mid = [op.node("Cast", ["x"], ["x16"], to=F16), _conv("x16", "w", None, "a"),
           op.node("Cast", ["a"], ["a32"], to=F32), op.node("Cast", ["a32"], ["b"], to=F16),
           _conv("b", "w2", None, "c"), op.node("Cast", ["c"], ["y"], to=F32)]
    m2 = _model(mid, "x", [1, 1, "h", "w"], F32, "y", [1, 1, "h", "w"], F32,
                [_half("w", w), _half("w2", w2)])
    assert claims(m2) == [[0, 1], [4, 5]]


# ---------------------------------------------------------------------------
# The fused node's MetaDef (activation input, initializers, outputs)
# ---------------------------------------------------------------------------

def test_run_boundary(fixtures):
    from arthip_amd.engine import run_boundary
    m = fixtures.get("ep_two_convs_one_input").model
    acts, consts, outs = run_boundary(m, [0, 1, 2])
    assert acts == ["x"] and outs == ["y"]
    assert consts == ["w1", "b1", "w2", "b2"]
    # A sub-run exports what the rest of the graph reads.
    acts, consts, outs = run_boundary(m, [0, 1])
    assert acts == ["x"] and consts == ["w1", "b1", "w2", "b2"] and outs == ["ca", "cb"]
    g = op.Graph(nodes=[op.node("Add", ["x1", "x2"], ["y"])],
                 inputs=[op.value_info("x1", F16, [1, 4, "h", "w"]),
                         op.value_info("x2", F16, [1, 4, "h", "w"])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"])])
    assert run_boundary(op.Model(graph=g), [0]) == (["x1", "x2"], [], ["y"])
    with pytest.raises(EngineError, match="increasing"):
        run_boundary(m, [1, 0])
    with pytest.raises(EngineError, match="empty"):
        run_boundary(m, [])


# ---------------------------------------------------------------------------
# Runs named by node keys, and the fused node's own graph
# ---------------------------------------------------------------------------

def _chain_after_prefix(order, cast_pair=False):
    """An unsupported prefix (Tanh on the input, and a Shape node beside it whose
    output is a second graph output), then the chain Conv -> Relu -> Conv that
    the EP claims. `order` permutes the node list among valid topological
    orders; `cast_pair` puts an fp16 -> fp32 -> fp16 Cast pair between the
    prefix and the chain (unclaimed: neither Cast touches the graph boundary)."""
    w1, w2 = kern(41, 8, 4), kern(42, 4, 8)
    tanh = op.node("Tanh", ["x"], ["xt"])
    shape = op.node("Shape", ["x"], ["shp"])
    head_in = "xt"
    casts = []
    if cast_pair:
        casts = [op.node("Cast", ["xt"], ["x32"], to=F32), op.node("Cast", ["x32"], ["x16"], to=F16)]
        head_in = "x16"
    chain = [_conv(head_in, "w1", None, "a"), op.node("Relu", ["a"], ["r"]),
             _conv("r", "w2", None, "y")]
    named = {"tanh": tanh, "shape": shape, "c1": chain[0], "relu": chain[1], "c2": chain[2]}
    nodes = []
    for key in order:
        nodes.append(named[key])
        if key == "tanh":
            nodes.extend(casts)
    g = op.Graph(nodes=nodes, name="prefix_chain",
                 initializers=[_half("w1", w1), _half("w2", w2)],
                 inputs=[op.value_info("x", F16, [1, 4, "h", "w"])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"]),
                          op.value_info("shp", op.INT64, [4])])
    return op.Model(graph=g, opset_imports=[("", 17)])


ORDERS = [["tanh", "shape", "c1", "relu", "c2"], ["shape", "tanh", "c1", "relu", "c2"],
          ["tanh", "c1", "relu", "c2", "shape"]]


def _runs_by_key(model):
    from arthip_amd.engine import node_keys
    return [node_keys(model, run) for run in claims(model)]


def _resolve(keys, model):
    """What an EP shim does with the keys: find each node in its own node list
    (ONNX Runtime's graph) by output name."""
    by_output = {}
    for i, n in enumerate(model.graph.nodes):
        for o in n.outputs:
            if o:
                by_output[o] = i
    return [by_output[k] for k in keys]


def test_runs_by_key_survive_node_order_and_removed_casts():
    """The same claimed run, named by keys, in every node order and with a Cast
    pair removed before it; its node positions change with all of these. Keys
    resolved in another serialization's node list select the same Conv, Relu,
    Conv; the positions of one serialization applied to another would not."""
    variants = [_chain_after_prefix(o) for o in ORDERS]
    variants += [_chain_after_prefix(o, cast_pair=True) for o in ORDERS[:2]]
    positions = [claims(m) for m in variants]
    assert positions == [[[2, 3, 4]], [[2, 3, 4]], [[1, 2, 3]], [[4, 5, 6]], [[4, 5, 6]]]
    keyed = [_runs_by_key(m) for m in variants]
    assert all(k == [["a", "r", "y"]] for k in keyed), keyed
    for src in variants:
        (keys,) = _runs_by_key(src)
        for dst in variants:
            picked = [dst.graph.nodes[i] for i in _resolve(keys, dst)]
            assert [n.op_type for n in picked] == ["Conv", "Relu", "Conv"]
            assert [n.outputs[0] for n in picked] == ["a", "r", "y"]
    # Positions do not carry over: the third order's run, applied to the first
    # order's node list, would pick the Shape node and drop the last Conv.
    wrong = [variants[0].graph.nodes[i] for i in positions[2][0]]
    assert [n.op_type for n in wrong] == ["Shape", "Conv", "Relu"]


def test_node_keys_errors():
    from arthip_amd.engine import node_keys
    m = _chain_after_prefix(ORDERS[0])
    assert node_keys(m, [0, 1]) == ["xt", "shp"]
    assert node_keys(m, []) == []
    with pytest.raises(EngineError, match="outside"):
        node_keys(m, [5])
    g = op.Graph(nodes=[op.node("Relu", ["x"], [""]), op.node("Relu", ["x"], ["y"])],
                 inputs=[op.value_info("x", F16, [1, 4, "h", "w"])],
                 outputs=[op.value_info("y", F16, [1, 4, "h", "w"])])
    with pytest.raises(EngineError, match="no output"):
        node_keys(op.Model(graph=g), [0])


@pytest.mark.parametrize("which", ["shipped", "prefix_chain", "fp32io"])
def test_fused_node_graph_is_claimed_whole(which, fixtures):
    """Compile works from the fused node's own graph: serialized on its own, with
    the initializers also listed as graph inputs, it is one claimed run of all
    its nodes with the same MetaDef as the run in the whole model."""
    from arthip_amd.engine import run_boundary
    if which == "shipped":
        m = op.load(GOLDEN / "ArtCNN_R8F64_fp16.onnx")
    elif which == "prefix_chain":
        m = _chain_after_prefix(ORDERS[1], cast_pair=True)
    else:
        m = op.load(fixtures.get("ep_conv_fp32io").model)
    (run,) = claims(m)
    sub = fused_node_graph(m, run)
    n = len(sub.graph.nodes)
    assert claims(sub) == [list(range(n))]
    assert run_boundary(sub, list(range(n))) == run_boundary(m, run)
