"""fp32 -> fp16 model conversion as the VapourSynth filter applies it at load
time with fp16=1 -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates src/vapoursynth/convert_float_to_float16.cpp:294-611 as hip.Model calls
it (src/vapoursynth/vs_hip.cpp:510-515: force_fp16_initializers=true, an empty
op block list, cast_input = cast_output = "the clip is fp32") for the ops of a
conv-chain model:
- every FLOAT initializer becomes FLOAT16 with the converter's own rounding
  (``half_no_subnormals``, lines 158-186);
- with cast_input, each FLOAT graph input keeps its type and a Cast to FLOAT16
  named ``graph_input_cast_<i>`` is put first, its consumers renamed (312-361);
  without, the input itself becomes FLOAT16;
- with cast_output, each FLOAT graph output is produced by an appended Cast to
  FLOAT from ``graph_output_cast_<i>`` (363-400); without, the output becomes
  FLOAT16;
- a Cast to FLOAT inside the graph becomes a Cast to FLOAT16 (470-480).
Node arithmetic itself is unchanged; ``oracle.model.run_model`` on the result
stores every activation as fp16.

Pins (tests/test_vs_cpu.py): ``half_no_subnormals`` against numpy's IEEE
float16 cast in the normal range and against the rule's fixed points (2^-14,
its predecessor, 65504, 65520, ties to even, NaN, inf); ``to_fp16`` against the
graph structure the converter's source describes.
"""

from __future__ import annotations

import copy

import numpy as np

from arthip_amd import onnx_proto as op

_MIN_NORMAL = np.float32(2.0 ** -14)


def half_no_subnormals(x) -> np.ndarray:
    """float32 -> float16: round to nearest even, |x| < 2^-14 -> signed zero,
    NaN and overflow -> signed inf (convert_float_to_float16.cpp:158-186)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = x.astype(np.float16)
    sign = np.signbit(x)
    zero = np.where(sign, np.float16(-0.0), np.float16(0.0))
    inf = np.where(sign, np.float16(-np.inf), np.float16(np.inf))
    h = np.where(np.abs(x) < _MIN_NORMAL, zero, h)
    return np.where(np.isnan(x), inf, h).astype(np.float16)


def to_fp16(model: op.Model, *, cast_input: bool, cast_output: bool) -> op.Model:
    m = copy.deepcopy(model)
    g = m.graph
    init_names = {t.name for t in g.initializers}
    for i, t in enumerate(g.initializers):
        if t.data_type == op.FLOAT:
            h = half_no_subnormals(t.to_numpy())
            g.initializers[i] = op.Tensor(name=t.name, dims=list(t.dims), data_type=op.FLOAT16,
                                          raw_data=h.tobytes())
    io_casts = set()
    head, tail = [], []
    if cast_input:
        fp32_in = [v for v in g.inputs if v.elem_type == op.FLOAT and v.name not in init_names]
        for i, v in enumerate(fp32_in):
            new = f"graph_input_cast_{i}"
            for n in g.nodes:
                n.inputs = [new if x == v.name else x for x in n.inputs]
            head.append(op.node("Cast", [v.name], [new], to=op.FLOAT16))
            io_casts.add(new)
    if cast_output:
        fp32_out = [v for v in g.outputs if v.elem_type == op.FLOAT]
        for i, v in enumerate(fp32_out):
            new = f"graph_output_cast_{i}"
            for n in g.nodes:
                n.outputs = [new if x == v.name else x for x in n.outputs]
            tail.append(op.node("Cast", [new], [v.name], to=op.FLOAT))
            io_casts.add(new)
    for n in g.nodes:
        if n.op_type == "Cast" and int(n.attr("to")) == op.FLOAT:
            n.attributes = [op.attr("to", op.FLOAT16) if a.name == "to" else a
                            for a in n.attributes]
    g.nodes = head + g.nodes + tail
    if not cast_input:
        for v in g.inputs:
            if v.elem_type == op.FLOAT and v.name not in init_names:
                v.elem_type = op.FLOAT16
    if not cast_output:
        for v in g.outputs:
            if v.elem_type == op.FLOAT:
                v.elem_type = op.FLOAT16
    return m
