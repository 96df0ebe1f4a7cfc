"""Synthetic ArtCNN-style models, written as fp16 ONNX with the package's own codec.

The benchmark workloads are random-initialised models of the ArtCNN family (no
checkpoints are available): 3x3 SAME convs with He-normal weights,
ReLU or SiLU, residual blocks, a global skip and a DepthToSpace(2) tail. All
builders are deterministic in their seed.

Config names follow the workloads the engine is measured on:
  c4f32        conv 1->32+ReLU, 2x conv 32->32+ReLU, conv 32->4, DepthToSpace(2)
  single64     one conv 64->64 + bias + ReLU (input 1x64xHxW)
  r8f64        conv 1->64; 8 x [conv 64->64+ReLU, conv 64->64, +skip];
               +global skip; conv 64->4; DepthToSpace(2)
  r16f96       the same with 16 blocks of 96 channels
  shipped_like the shipped luma model's structure (SiLU, 3-conv blocks, one
               more conv before the global skip, Clip(0,1) tail), random weights
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import onnx_proto as op

OPSET = 17


def he_normal(rng: np.random.Generator, m: int, c: int) -> np.ndarray:
    """He-normal 3x3 kernel N(0, 2/(9c)), drawn in fp32, stored as fp16."""
    return (rng.standard_normal((m, c, 3, 3), dtype=np.float32) *
            np.float32(np.sqrt(2.0 / (9 * c)))).astype(np.float16)


@dataclass
class ModelSpec:
    """What a builder produced: the model plus the facts tests and bench need."""

    model: op.Model
    name: str
    in_channels: int
    out_channels: int
    scale: int
    convs: list  # (cin, cout) per conv in execution order, for FLOP/byte counting
    skips_per_conv: list  # residual inputs fused into each conv (0, 1 or 2)
    conv_inputs: list | None = None  # input tensor name per conv
    skip_names: list | None = None  # residual input tensor names per conv

    def bytes(self) -> bytes:
        return op.encode_model(self.model)

    def save(self, path) -> None:
        op.save(self.model, path)


class _Builder:
    def __init__(self, seed: int, bias: str = "zero", io_fp32: bool = False):
        self.rng = np.random.default_rng(seed)
        self.bias = bias
        self.io_fp32 = io_fp32
        self.nodes: list[op.Node] = []
        self.inits: list[op.Tensor] = []
        self.convs: list = []
        self.skips: list = []
        self.conv_in: list = []
        self.skip_names: list = []
        self.k = 0

    def conv(self, x: str, cin: int, cout: int, act: str | None = None) -> str:
        i = self.k
        self.k += 1
        w = he_normal(self.rng, cout, cin)
        self.inits.append(op.tensor(f"w{i}", w))
        ins = [x, f"w{i}"]
        if self.bias == "zero":
            b = np.zeros(cout, np.float16)
        else:
            b = self.rng.uniform(-0.1, 0.1, cout).astype(np.float16)
        self.inits.append(op.tensor(f"b{i}", b))
        ins.append(f"b{i}")
        y = f"conv{i}"
        self.nodes.append(op.node("Conv", ins, [y], kernel_shape=[3, 3], pads=[1, 1, 1, 1],
                                  strides=[1, 1], dilations=[1, 1], group=1))
        self.convs.append((cin, cout))
        self.skips.append(0)
        self.conv_in.append(x)
        self.skip_names.append([])
        if act == "relu":
            self.nodes.append(op.node("Relu", [y], [f"relu{i}"]))
            y = f"relu{i}"
        elif act == "silu":
            self.nodes.append(op.node("Sigmoid", [y], [f"sig{i}"]))
            self.nodes.append(op.node("Mul", [y, f"sig{i}"], [f"silu{i}"]))
            y = f"silu{i}"
        return y

    def add(self, a: str, b: str, name: str) -> str:
        self.nodes.append(op.node("Add", [a, b], [name]))
        self.skips[-1] += 1
        self.skip_names[-1].append(b)
        return name

    def finish(self, x_in: str, y: str, cin: int, cout: int, out_name="y") -> op.Model:
        nodes = list(self.nodes)
        in_t = op.FLOAT if self.io_fp32 else op.FLOAT16
        if self.io_fp32:
            nodes.insert(0, op.node("Cast", ["x"], [x_in], to=op.FLOAT16))
            nodes.append(op.node("Cast", [y], [out_name], to=op.FLOAT))
            y = out_name
        elif y != out_name:
            # rename the last output to the graph output name
            last = nodes[-1]
            last.outputs = [out_name if o == y else o for o in last.outputs]
            y = out_name
        g = op.Graph(nodes=nodes, name="artcnn", initializers=self.inits,
                     inputs=[op.value_info("x", in_t, [1, cin, "H", "W"])],
                     outputs=[op.value_info(y, in_t, [1, cout, "H2", "W2"])])
        return op.Model(graph=g, opset_imports=[("", OPSET)])


def artcnn(blocks: int, filters: int, *, convs_per_block: int = 2, act: str = "relu",
           in_ch: int = 1, scale: int = 2, out_ch: int = 1, seed: int = 0, bias: str = "zero",
           global_skip: bool = True, pre_skip_conv: bool = False, clip: tuple | None = None,
           io_fp32: bool = False, name: str = "artcnn") -> ModelSpec:
    """ArtCNN-style residual upscaler.

    head conv in_ch->F; blocks x [conv+act (convs_per_block-1 times), conv, +skip];
    [conv] (pre_skip_conv); +head (global_skip); conv F->out_ch*scale^2;
    DepthToSpace(scale, DCR); [Clip].
    """
    b = _Builder(seed, bias, io_fp32)
    x = "xh" if io_fp32 else "x"
    head = b.conv(x, in_ch, filters)
    h = head
    for i in range(blocks):
        t = h
        for _ in range(convs_per_block - 1):
            t = b.conv(t, filters, filters, act)
        t = b.conv(t, filters, filters)
        h = b.add(t, h, f"blk{i}")
    if pre_skip_conv:
        h = b.conv(h, filters, filters)
    if global_skip:
        h = b.add(h, head, "gskip")
    t = b.conv(h, filters, out_ch * scale * scale)
    if scale > 1:
        b.nodes.append(op.node("DepthToSpace", [t], ["d2s"], blocksize=scale, mode="DCR"))
        t = "d2s"
    if clip is not None:
        lo = op.tensor("clip_lo", np.array(clip[0], np.float16))
        hi = op.tensor("clip_hi", np.array(clip[1], np.float16))
        b.inits += [lo, hi]
        b.nodes.append(op.node("Clip", [t, "clip_lo", "clip_hi"], ["clipped"]))
        t = "clipped"
    model = b.finish(x, t, in_ch, out_ch)
    return ModelSpec(model, name, in_ch, out_ch, scale, b.convs, b.skips, b.conv_in, b.skip_names)


def c4f32(seed: int = 0) -> ModelSpec:
    b = _Builder(seed)
    t = b.conv("x", 1, 32, "relu")
    t = b.conv(t, 32, 32, "relu")
    t = b.conv(t, 32, 32, "relu")
    t = b.conv(t, 32, 4)
    b.nodes.append(op.node("DepthToSpace", [t], ["d2s"], blocksize=2, mode="DCR"))
    model = b.finish("x", "d2s", 1, 1)
    return ModelSpec(model, "c4f32", 1, 1, 2, b.convs, b.skips, b.conv_in, b.skip_names)


def single64(seed: int = 0) -> ModelSpec:
    b = _Builder(seed, bias="uniform")
    t = b.conv("x", 64, 64, "relu")
    model = b.finish("x", t, 64, 64)
    return ModelSpec(model, "single64", 64, 64, 1, b.convs, b.skips, b.conv_in, b.skip_names)


def r8f64(seed: int = 0, **kw) -> ModelSpec:
    return artcnn(8, 64, seed=seed, name="r8f64", **kw)


def r16f96(seed: int = 0, **kw) -> ModelSpec:
    return artcnn(16, 96, seed=seed, name="r16f96", **kw)


def shipped_like(seed: int = 0, **kw) -> ModelSpec:
    return artcnn(8, 64, convs_per_block=3, act="silu", pre_skip_conv=True, clip=(0.0, 1.0),
                  seed=seed, bias="uniform", name="shipped_like", **kw)


CONFIGS = {
    "c4f32": (c4f32, (1, 1, 540, 960)),
    "single64": (single64, (1, 64, 1080, 1920)),
    "r8f64": (r8f64, (1, 1, 1080, 1920)),
    "r16f96": (r16f96, (1, 1, 1080, 1920)),
    "r8f64_4k_x2": (r8f64, (2, 1, 2160, 3840)),
}


def synthetic_input(shape, seed: int = 1, kind: str = "uniform") -> np.ndarray:
    """Seeded NCHW fp16 input: uniform [0, 1) luma, or normal(0, 0.5) activations."""
    rng = np.random.default_rng(seed)
    if kind == "normal":
        x = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.5)
    else:
        x = rng.random(shape, dtype=np.float32)
    return x.astype(np.float16)


def work_per_frame(spec: ModelSpec, n: int, h: int, w: int) -> dict:
    """Algorithmic work of one pass at input (n, h, w):

    flops_direct  sum over convs of 2*9*Cin*Cout*N*H*W
    flops_wino    Winograd-executed convs (Cin > 1) at 16/36 of that, head conv direct
    bytes         layer-at-a-time compulsory HBM traffic: each conv reads its input
                  and residual inputs and writes its output once (fp16), plus the
                  fp16 weights; the DepthToSpace tail is fused into the last conv.
    """
    px = n * h * w
    fd = fw = 0.0
    byts = 0.0
    for (cin, cout), nskip in zip(spec.convs, spec.skips_per_conv):
        f = 2.0 * 9 * cin * cout * px
        fd += f
        fw += f * (16.0 / 36.0) if cin > 1 else f
        byts += 2.0 * px * (cin + cout * (1 + nskip)) + 2.0 * 9 * cin * cout
    return {"flops_direct": fd, "flops_wino": fw, "bytes": byts}


def widen_to_fp32(spec: ModelSpec, name: str | None = None) -> ModelSpec:
    """The same network as an all-fp32 ONNX model: fp32 initializers (exact
    widenings of the fp16 weights), fp32 graph IO and no Cast nodes.

    This is the form the reference's VapourSynth plugin converts to fp16 before
    building (``fp16=1``; convert_float_to_float16.cpp:294-611). The engine
    takes it directly: weights are rounded to fp16 when they are packed and the
    boundary converts fp32 <-> fp16, so an fp32 model runs exactly the fp16
    network with fp32 IO."""
    g = spec.model.graph
    boundary = {n.outputs[0]: n.inputs[0] for n in g.nodes if n.op_type == "Cast"}
    nodes = []
    for n in g.nodes:
        if n.op_type == "Cast":
            continue
        ins = ["x" if boundary.get(i) == "x" else i for i in n.inputs]
        nodes.append(op.Node(n.op_type, ins, list(n.outputs), n.name, n.domain, list(n.attributes)))
    out_name = g.outputs[0].name
    if out_name in boundary:  # the graph output was a Cast of `src`
        src = boundary[out_name]
        for n in nodes:
            n.outputs = [out_name if o == src else o for o in n.outputs]
    inits = []
    for t in g.initializers:
        a = t.to_numpy()
        inits.append(op.tensor(t.name, a.astype(np.float32) if a.dtype == np.float16 else a))
    gi, go = g.inputs[0], g.outputs[0]
    graph = op.Graph(nodes=nodes, name=g.name, initializers=inits,
                     inputs=[op.value_info(gi.name, op.FLOAT, gi.shape)],
                     outputs=[op.value_info(go.name, op.FLOAT, go.shape)])
    model = op.Model(graph=graph, opset_imports=list(spec.model.opset_imports))
    return ModelSpec(model, name or spec.name + "_fp32", spec.in_channels, spec.out_channels,
                     spec.scale, list(spec.convs), list(spec.skips_per_conv),
                     spec.conv_inputs, spec.skip_names)
