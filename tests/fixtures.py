"""Tiny ONNX fixtures equivalent to the reference suite's (one engine property each).

Regenerates, with this repo's own ONNX writer, the fixture set that
tests/correctness/harness/modelgen.py builds with the ``onnx`` package (absent
here): same names, same seeds, weights ``RandomState(seed).uniform(-0.5, 0.5)``
stored as fp16 (modelgen.py:124-125), biases ``linspace(-0.1, 0.1)``
(modelgen.py:128-129), and the same graphs (modelgen.py:137-530).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

from arthip_amd import onnx_proto as op

OPSET = 17


@dataclass(frozen=True)
class Fixture:
    name: str
    model: Path
    input_channels: int
    output_channels: int
    weights: np.ndarray | None = None  # fp16, as stored in the model
    bias: np.ndarray | None = None
    blocksize: int = 0
    fp32_io: bool = False


def kern(seed: int, m: int, c: int, k: int = 3) -> np.ndarray:
    return np.random.RandomState(seed).uniform(-0.5, 0.5, (m, c, k, k)).astype(np.float32)


def linspace(m: int, lo: float = -0.1, hi: float = 0.1) -> np.ndarray:
    return np.linspace(lo, hi, m).astype(np.float32)


def _half(name, a):
    return op.tensor(name, np.asarray(a, np.float16))


def _float(name, a):
    return op.tensor(name, np.asarray(a, np.float32))


def _conv(x, w, b, out, *, kernel=3, pads=(1, 1, 1, 1)):
    return op.node("Conv", [x, w] + ([b] if b else []), [out], kernel_shape=[kernel, kernel],
                   pads=list(pads), strides=[1, 1], dilations=[1, 1], group=1)


def _model(nodes, in_name, in_shape, in_type, out_name, out_shape, out_type, inits, inputs=None):
    g = op.Graph(nodes=nodes, name="fixture", initializers=inits,
                 inputs=inputs or [op.value_info(in_name, in_type, in_shape)],
                 outputs=[op.value_info(out_name, out_type, out_shape)])
    return op.Model(graph=g, opset_imports=[("", OPSET)])


def fused_node_graph(model, run):
    """The fused node's own graph as ONNX Runtime hands it to Compile
    (FusedNodeAndGraph::filtered_graph) and as the EP shim serializes it: the
    run's nodes; as inputs the MetaDef inputs (the activation, then the
    initializers); the initializers; the MetaDef output."""
    from arthip_amd.engine import run_boundary
    acts, consts, outs = run_boundary(model, run)
    g = model.graph
    inits = {t.name: t for t in g.initializers}
    declared = {v.name: v for v in list(g.inputs) + list(g.outputs)}

    def info(name):
        if name in inits:
            t = inits[name]
            return op.value_info(name, t.data_type, list(t.dims))
        if name in declared:
            return declared[name]
        return op.value_info(name, op.FLOAT16, None)

    sub = op.Graph(nodes=[g.nodes[i] for i in run], name="fused",
                   initializers=[inits[c] for c in consts],
                   inputs=[info(n) for n in acts + consts], outputs=[info(n) for n in outs])
    return op.Model(graph=sub, opset_imports=model.opset_imports)


class FixtureSet:
    def __init__(self, out: Path):
        self.out = Path(out)
        self.out.mkdir(parents=True, exist_ok=True)
        self._cache: dict[str, Fixture] = {}

    def _save(self, model: op.Model, name: str) -> Path:
        p = self.out / f"{name}.onnx"
        op.save(model, p)
        return p

    def get(self, name: str) -> Fixture:
        if name not in self._cache:
            self._cache[name] = getattr(self, "_" + name)()
        return self._cache[name]

    # -- single convs (modelgen.py:137-217) --------------------------------------
    def _single(self, name, *, m, c, seed, bias="full", kernel=3, pads=(1, 1, 1, 1),
                external=False) -> Fixture:
        w = kern(seed, m, c, kernel)
        wt = _half("w", w)
        if external:
            wt.raw_data = b""
            wt.data_location = 1
            wt.external_data = [("location", f"{name}.bin")]
        inits = [wt]
        fields = {"weights": w.astype(np.float16)}
        bname = None
        if bias != "none":
            blen = m if bias == "full" else int(bias)
            b = linspace(blen)
            inits.append(_half("b", b))
            bname = "b"
            if blen == m:
                fields["bias"] = b.astype(np.float16)
        node = _conv("x", "w", bname, "y", kernel=kernel, pads=pads)
        model = _model([node], "x", [1, c, "h", "w"], op.FLOAT16, "y", [1, m, "h", "w"],
                       op.FLOAT16, inits)
        return Fixture(name, self._save(model, name), c, m, **fields)

    def _conv_c4m4(self):
        return self._single("conv_c4m4", m=4, c=4, seed=11)

    def _conv_c4m8(self):
        return self._single("conv_c4m8", m=8, c=4, seed=12)

    def _conv_c4m64(self):
        return self._single("conv_c4m64", m=64, c=4, seed=13)

    def _conv_c1m8(self):
        return self._single("conv_c1m8", m=8, c=1, seed=21)

    def _conv_m128(self):
        return self._single("conv_m128", m=128, c=4, seed=51, bias="none")

    def _conv_m160(self):
        return self._single("conv_m160", m=160, c=4, seed=52, bias="none")

    def _conv_c128(self):
        return self._single("conv_c128", m=4, c=128, seed=53, bias="none")

    def _conv_1x1(self):
        return self._single("conv_1x1", m=4, c=4, seed=31, bias="none", kernel=1)

    def _conv_short_bias(self):
        return self._single("conv_short_bias", m=4, c=4, seed=41, bias=2)

    def _conv_external(self):
        return self._single("conv_external", m=4, c=4, seed=95, bias="none", external=True)

    def _conv_pads_asym(self):
        return self._single("conv_pads_asym", m=4, c=4, seed=33, bias="none", pads=(1, 0, 1, 0))

    # -- typed fp16 initializers (modelgen.py:224-249) ----------------------------
    def _identity(self, name, typed):
        ident = np.zeros((1, 1, 3, 3), np.float32)
        ident[0, 0, 1, 1] = 1.0
        init = op.tensor("w", ident.astype(np.float16), typed_half=typed)
        model = _model([_conv("x", "w", None, "y")], "x", [1, 1, "h", "w"], op.FLOAT16,
                       "y", [1, 1, "h", "w"], op.FLOAT16, [init])
        return Fixture(name, self._save(model, name), 1, 1, weights=ident.astype(np.float16))

    def _identity_raw(self):
        return self._identity("identity_raw", False)

    def _identity_typed_half(self):
        return self._identity("identity_typed_half", True)

    # -- binary operands (modelgen.py:256-281) ------------------------------------
    def _add_const(self):
        w = kern(61, 4, 4)
        nodes = [_conv("x", "w", None, "raw"), op.node("Add", ["raw", "k"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w), _float("k", np.full((1, 1, 1, 1), 0.25))])
        return Fixture("add_const", self._save(model, "add_const"), 4, 4,
                       weights=w.astype(np.float16))

    def _add_broadcast(self):
        w, w2 = kern(71, 4, 4), kern(72, 1, 4)
        nodes = [_conv("x", "w", None, "a"), _conv("x", "w2", None, "b"),
                 op.node("Add", ["a", "b"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w), _half("w2", w2)])
        return Fixture("add_broadcast", self._save(model, "add_broadcast"), 4, 4,
                       weights=w.astype(np.float16))

    # -- DepthToSpace (modelgen.py:288-357) ----------------------------------------
    def _dts(self, name, b):
        m = b * b
        w, bias = kern(80 + b, m, 1), linspace(m, -0.05, 0.05)
        nodes = [_conv("x", "w", "b", "raw"),
                 op.node("DepthToSpace", ["raw"], ["sq"], blocksize=b, mode="DCR"),
                 op.node("Cast", ["sq"], ["y"], to=op.FLOAT)]
        model = _model(nodes, "x", [1, 1, "h", "w"], op.FLOAT16, "y", [1, 1, "h", "w"],
                       op.FLOAT, [_half("w", w), _half("b", bias)])
        return Fixture(name, self._save(model, name), 1, 1, weights=w.astype(np.float16),
                       bias=bias.astype(np.float16), blocksize=b, fp32_io=True)

    def _dts_b1(self):
        return self._dts("dts_b1", 1)

    def _dts_b2(self):
        return self._dts("dts_b2", 2)

    def _dts_b3(self):
        return self._dts("dts_b3", 3)

    def _dts_multi(self, name, b, cout, fp32_out):
        m = cout * b * b
        w, bias = kern(90 + b * 10 + cout, m, 1), linspace(m, -0.05, 0.05)
        nodes = [_conv("x", "w", "b", "raw"),
                 op.node("DepthToSpace", ["raw"], ["sq"], blocksize=b, mode="DCR")]
        if fp32_out:
            nodes.append(op.node("Cast", ["sq"], ["y"], to=op.FLOAT))
            out, ot = "y", op.FLOAT
        else:
            out, ot = "sq", op.FLOAT16
        model = _model(nodes, "x", [1, 1, "h", "w"], op.FLOAT16, out, [1, cout, "h", "w"], ot,
                       [_half("w", w), _half("b", bias)])
        return Fixture(name, self._save(model, name), 1, cout, weights=w.astype(np.float16),
                       bias=bias.astype(np.float16), blocksize=b, fp32_io=fp32_out)

    def _dts_multi_b2(self):
        return self._dts_multi("dts_multi_b2", 2, 2, True)

    def _dts_multi_b2_f16(self):
        return self._dts_multi("dts_multi_b2_f16", 2, 2, False)

    def _dts_multi_b3(self):
        return self._dts_multi("dts_multi_b3", 3, 2, True)

    # -- fusion with shared intermediates (modelgen.py:364-408) ---------------------
    def _silu_shared(self):
        w, b = kern(63, 4, 4), linspace(4)
        nodes = [_conv("x", "w", "b", "raw"), op.node("Sigmoid", ["raw"], ["sig"]),
                 op.node("Mul", ["raw", "sig"], ["z"]), op.node("Add", ["raw", "z"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w), _half("b", b)])
        return Fixture("silu_shared", self._save(model, "silu_shared"), 4, 4,
                       weights=w.astype(np.float16), bias=b.astype(np.float16))

    def _add_shared_conv_out(self):
        w, b = (kern(64, 4, 4) * 0.2).astype(np.float32), linspace(4)
        nodes = [_conv("x", "w", "b", "a"), _conv("a", "w", "b", "bb"),
                 op.node("Add", ["a", "bb"], ["s"]), op.node("Mul", ["bb", "s"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w), _half("b", b)])
        return Fixture("add_shared_conv_out", self._save(model, "add_shared_conv_out"), 4, 4,
                       weights=w.astype(np.float16), bias=b.astype(np.float16))

    # -- Clip bounds (modelgen.py:429-455) ------------------------------------------
    def _clip_no_bounds(self):
        w, b = kern(34, 4, 4), np.full((4,), 2.0, np.float32)
        nodes = [_conv("x", "w", "b", "raw"), op.node("Clip", ["raw"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w), _half("b", b)])
        return Fixture("clip_no_bounds", self._save(model, "clip_no_bounds"), 4, 4,
                       weights=w.astype(np.float16), bias=b.astype(np.float16))

    def _clip_dynamic_bound(self):
        w = kern(35, 4, 4)
        nodes = [_conv("x", "w", None, "raw"), op.node("Clip", ["raw", "raw"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w", w)])
        return Fixture("clip_dynamic_bound", self._save(model, "clip_dynamic_bound"), 4, 4,
                       weights=w.astype(np.float16))

    # -- partitions / fp32 IO (modelgen.py:462-530) ----------------------------------
    def _ep_two_convs_one_input(self):
        w1, w2 = kern(81, 4, 4), kern(82, 4, 4)
        b1, b2 = linspace(4), linspace(4, -0.2, 0.2)
        nodes = [_conv("x", "w1", "b1", "ca"), _conv("x", "w2", "b2", "cb"),
                 op.node("Add", ["ca", "cb"], ["y"])]
        model = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"],
                       op.FLOAT16, [_half("w1", w1), _half("b1", b1), _half("w2", w2),
                                    _half("b2", b2)])
        return Fixture("ep_two_convs_one_input", self._save(model, "ep_two_convs_one_input"),
                       4, 4, weights=w1.astype(np.float16), bias=b1.astype(np.float16))

    def _identity_fp32io(self):
        ident = np.zeros((1, 1, 3, 3), np.float32)
        ident[0, 0, 1, 1] = 1.0
        nodes = [op.node("Cast", ["x"], ["xh"], to=op.FLOAT16), _conv("xh", "w", None, "raw"),
                 op.node("Cast", ["raw"], ["y"], to=op.FLOAT)]
        model = _model(nodes, "x", [1, 1, "h", "w"], op.FLOAT, "y", [1, 1, "h", "w"], op.FLOAT,
                       [_half("w", ident)])
        return Fixture("identity_fp32io", self._save(model, "identity_fp32io"), 1, 1,
                       weights=ident.astype(np.float16), fp32_io=True)

    def _ep_conv_fp32io(self):
        w, b = kern(5, 1, 1), linspace(1)
        nodes = [op.node("Cast", ["x"], ["xh"], to=op.FLOAT16), _conv("xh", "w", "b", "raw"),
                 op.node("Cast", ["raw"], ["y"], to=op.FLOAT)]
        model = _model(nodes, "x", [1, 1, "h", "w"], op.FLOAT, "y", [1, 1, "h", "w"], op.FLOAT,
                       [_half("w", w), _half("b", b)])
        return Fixture("ep_conv_fp32io", self._save(model, "ep_conv_fp32io"), 1, 1,
                       weights=w.astype(np.float16), bias=b.astype(np.float16), fp32_io=True)

    def _multi_in_out(self):
        """C=3 fp16 NCHW input, 2-channel NCHW output (layout conversion both ways)."""
        w, b = kern(77, 2, 3), linspace(2)
        model = _model([_conv("x", "w", "b", "y")], "x", [1, 3, "h", "w"], op.FLOAT16, "y",
                       [1, 2, "h", "w"], op.FLOAT16, [_half("w", w), _half("b", b)])
        return Fixture("multi_in_out", self._save(model, "multi_in_out"), 3, 2,
                       weights=w.astype(np.float16), bias=b.astype(np.float16))
