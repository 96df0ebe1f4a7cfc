#include "graph.h"

#include <algorithm>
#include <cstring>
#include <functional>
#include <unordered_set>

#include "conv_args.h"
#include "half.h"

namespace arthip {

const char* OpKindName(OpKind k) {
  switch (k) {
    case OpKind::Conv: return "Conv";
    case OpKind::Sigmoid: return "Sigmoid";
    case OpKind::Relu: return "Relu";
    case OpKind::Mul: return "Mul";
    case OpKind::Add: return "Add";
    case OpKind::Clip: return "Clip";
    case OpKind::DepthToSpace: return "DepthToSpace";
  }
  return "?";
}

int MaxConvInputChannels() { return 96; }
int MaxConvOutputChannels() { return 128; }

float WeightAt(const Weight& w, size_t idx) {
  if (w.dtype == onnx::kFloat) {
    if ((idx + 1) * 4 > w.data.size()) return 0.0f;
    float v;
    std::memcpy(&v, w.data.data() + idx * 4, 4);
    return v;
  }
  if (w.dtype == onnx::kFloat16) {
    if ((idx + 1) * 2 > w.data.size()) return 0.0f;
    uint16_t b;
    std::memcpy(&b, w.data.data() + idx * 2, 2);
    return f16_to_f32(b);
  }
  return 0.0f;
}

namespace {

int64_t Numel(const std::vector<int64_t>& d) {
  int64_t n = 1;
  for (int64_t v : d) n *= v;
  return n;
}

// Initializer -> Weight, keeping the declared dtype. FLOAT16 values stored in
// int32_data are 16-bit bit patterns, not numbers (hip_engine.cc:46-112).
bool Materialize(const onnx::Tensor& t, Weight& w, std::string& error) {
  w.dtype = t.data_type;
  w.dims = t.dims;
  w.data.clear();
  if (t.data_location == 1 || t.has_external_data) {
    error = "initializer '" + t.name + "' uses external data, which is not supported";
    return false;
  }
  if (!t.raw_data.empty()) {
    if (onnx::DtypeSize(t.data_type) == 0) {
      error = "initializer '" + t.name + "' has an unsupported dtype";
      return false;
    }
    w.data.assign(t.raw_data.begin(), t.raw_data.end());
    return true;
  }
  if (!t.float_data.empty()) {
    if (t.data_type != onnx::kFloat) {
      error = "initializer '" + t.name + "' has float_data with a non-FLOAT dtype";
      return false;
    }
    w.data.resize(t.float_data.size() * 4);
    std::memcpy(w.data.data(), t.float_data.data(), w.data.size());
  } else if (!t.double_data.empty()) {
    if (t.data_type != onnx::kDouble) {
      error = "initializer '" + t.name + "' has double_data with a non-DOUBLE dtype";
      return false;
    }
    w.data.resize(t.double_data.size() * 8);
    std::memcpy(w.data.data(), t.double_data.data(), w.data.size());
  } else if (!t.int32_data.empty()) {
    const size_t es = onnx::DtypeSize(t.data_type);
    if (es == 0) {
      error = "initializer '" + t.name + "' has an unsupported dtype";
      return false;
    }
    w.data.resize(t.int32_data.size() * es);
    for (size_t k = 0; k < t.int32_data.size(); ++k) {
      const uint32_t v = static_cast<uint32_t>(t.int32_data[k]);
      std::memcpy(w.data.data() + k * es, &v, es);
    }
  } else if (!t.int64_data.empty()) {
    w.data.resize(t.int64_data.size() * 8);
    std::memcpy(w.data.data(), t.int64_data.data(), w.data.size());
  }
  return true;
}

}  // namespace

bool BuildGraph(const onnx::Model& model, Graph& g, std::string& error,
                const BuildOptions& opts) {
  g = Graph();
  const onnx::Graph& og = model.graph;

  for (size_t i = 0; i < og.initializers.size(); ++i) {
    const auto& t = og.initializers[i];
    if (t.name.empty()) {
      error = "initializer #" + std::to_string(i) + " has no name";
      return false;
    }
    Weight& w = g.weights[t.name];
    if (!Materialize(t, w, error)) return false;
    if (opts.fp16 && w.dtype == onnx::kFloat) {
      const size_t n = w.data.size() / 4;
      std::vector<uint8_t> h(n * 2);
      for (size_t k = 0; k < n; ++k) {
        float f;
        std::memcpy(&f, w.data.data() + 4 * k, 4);
        const uint16_t b = f32_to_f16_no_subnormals(f);
        std::memcpy(h.data() + 2 * k, &b, 2);
      }
      w.data.swap(h);
      w.dtype = onnx::kFloat16;
    }
  }

  // The activation input is the first graph input that is not an initializer
  // (older IR versions also list initializers as graph inputs).
  const onnx::ValueInfo* gin = nullptr;
  for (const auto& vi : og.inputs)
    if (!g.weights.count(vi.name)) {
      gin = &vi;
      break;
    }
  if (gin == nullptr || og.outputs.empty()) {
    error = "model must have at least one input and output";
    return false;
  }
  const onnx::ValueInfo& gout = og.outputs[0];
  g.input_name = gin->name;
  g.output_name = gout.name;

  // Consumer lists by tensor name.
  std::unordered_map<std::string, std::vector<int>> consumers;
  for (int i = 0; i < static_cast<int>(og.nodes.size()); ++i)
    for (const auto& in : og.nodes[i].inputs)
      if (!in.empty()) consumers[in].push_back(i);

  // Boundary Casts (fp32 graph IO around an fp16 body) fold into the IO
  // conversion; bare fp32 IO is handled the same way (hip_engine.cc:338-373).
  std::vector<bool> consumed(og.nodes.size(), false);
  const bool keep32 = !opts.fp16 || opts.keep_io_fp32;
  if (gin->elem_type == onnx::kFloat) {
    g.input_fp32 = keep32;
    for (int i = 0; i < static_cast<int>(og.nodes.size()); ++i) {
      const auto& n = og.nodes[i];
      if (n.op_type == "Cast" && !n.inputs.empty() && n.inputs[0] == g.input_name &&
          !n.outputs.empty()) {
        g.input_name = n.outputs[0];
        consumed[i] = true;
        break;
      }
    }
  }
  if (gout.elem_type == onnx::kFloat) {
    g.output_fp32 = keep32;
    for (int i = 0; i < static_cast<int>(og.nodes.size()); ++i) {
      const auto& n = og.nodes[i];
      if (n.op_type == "Cast" && !n.outputs.empty() && n.outputs[0] == g.output_name &&
          !n.inputs.empty()) {
        g.output_name = n.inputs[0];
        consumed[i] = true;
        break;
      }
    }
  }

  auto clip_scalar = [&](const std::string& name, float& dst) -> bool {
    if (name.empty()) return true;  // omitted bound keeps +/-inf
    auto it = g.weights.find(name);
    if (it == g.weights.end()) {
      error = "Clip bound '" + name +
              "' is not an initializer; dynamic Clip bounds are not supported";
      return false;
    }
    const Weight& w = it->second;
    if (w.data.empty()) return true;
    if (w.dtype == onnx::kFloat && w.data.size() >= 4) {
      std::memcpy(&dst, w.data.data(), 4);
      return true;
    }
    if (w.dtype == onnx::kFloat16 && w.data.size() >= 2) {
      uint16_t b;
      std::memcpy(&b, w.data.data(), 2);
      dst = f16_to_f32(b);
      return true;
    }
    if (w.dtype == onnx::kDouble && w.data.size() >= 8) {
      double d;
      std::memcpy(&d, w.data.data(), 8);
      dst = static_cast<float>(d);
      return true;
    }
    error = "Clip bound initializer '" + name + "' has an unsupported dtype or truncated storage";
    return false;
  };

  // ---- lower each node to an Op
  for (size_t ni = 0; ni < og.nodes.size(); ++ni) {
    if (consumed[ni]) continue;
    const onnx::Node& n = og.nodes[ni];
    if (n.outputs.empty() || n.outputs[0].empty()) continue;
    auto in = [&](size_t i) -> std::string { return i < n.inputs.size() ? n.inputs[i] : ""; };
    if (!n.domain.empty() && n.domain != "ai.onnx") {
      error = "unsupported op '" + n.domain + "::" + n.op_type + "' in fused graph";
      return false;
    }
    Op op;
    op.out = n.outputs[0];
    if (n.op_type == "Conv") {
      op.kind = OpKind::Conv;
      op.in0 = in(0);
      op.weight = in(1);
      op.bias = in(2);
      if (op.in0.empty() || op.weight.empty()) {
        error = "Conv missing inputs";
        return false;
      }
      int64_t sh = 1, sw = 1, dh = 1, dw = 1, group = 1, ph = 0, pw = 0;
      if (auto a = n.attr("strides"); a && a->ints.size() >= 2) sh = a->ints[0], sw = a->ints[1];
      if (auto a = n.attr("dilations"); a && a->ints.size() >= 2) dh = a->ints[0], dw = a->ints[1];
      if (auto a = n.attr("group")) group = a->i;
      if (auto a = n.attr("auto_pad")) {
        if (a->s == "SAME_UPPER" || a->s == "SAME_LOWER") {
          ph = pw = 1;
        } else if (a->s != "VALID" && a->s != "NOTSET") {
          error = "unsupported Conv auto_pad '" + a->s + "'";
          return false;
        }
      }
      // ONNX pads are [top, left, bottom, right]: only all-ones is the
      // symmetric 1-padding the kernels implement (hip_engine.cc:410-433).
      if (auto a = n.attr("pads"); a && !a->ints.empty()) {
        if (a->ints.size() != 4 || a->ints[0] != 1 || a->ints[1] != 1 || a->ints[2] != 1 ||
            a->ints[3] != 1) {
          error = "unsupported Conv pads (only symmetric 1-padding on both axes is supported)";
          return false;
        }
        ph = pw = 1;
      }
      if (sh != 1 || sw != 1 || dh != 1 || dw != 1 || ph != 1 || pw != 1 || group != 1) {
        error = "unsupported Conv configuration (only 3x3 stride 1, pad 1 supported)";
        return false;
      }
      auto wit = g.weights.find(op.weight);
      if (wit == g.weights.end()) {
        error = "expected initializer '" + op.weight + "' was not found";
        return false;
      }
      const Weight& w = wit->second;
      if (w.dims.size() != 4) {
        error = "Conv weight '" + op.weight + "' must be a rank-4 tensor";
        return false;
      }
      if (w.dims[2] != 3 || w.dims[3] != 3) {
        error = "Conv weight '" + op.weight + "' must be 3x3 (got " + std::to_string(w.dims[2]) +
                "x" + std::to_string(w.dims[3]) + ")";
        return false;
      }
      if (w.dims[0] <= 0 || w.dims[1] <= 0) {
        error = "Conv weight '" + op.weight + "' has a non-positive channel count";
        return false;
      }
      if (w.dims[0] > MaxConvOutputChannels()) {
        error = "conv supports at most " + std::to_string(MaxConvOutputChannels()) +
                " output channels (got " + std::to_string(w.dims[0]) + ")";
        return false;
      }
      if (w.dims[1] > MaxConvInputChannels()) {
        error = "conv supports at most " + std::to_string(MaxConvInputChannels()) +
                " input channels (got " + std::to_string(w.dims[1]) + ")";
        return false;
      }
      if (w.dtype != onnx::kFloat && w.dtype != onnx::kFloat16) {
        error = "Conv weight '" + op.weight + "' has unsupported dtype " + std::to_string(w.dtype);
        return false;
      }
      const size_t need = static_cast<size_t>(Numel(w.dims)) * onnx::DtypeSize(w.dtype);
      if (w.data.size() < need) {
        error = "Conv weight '" + op.weight + "' storage is truncated (" +
                std::to_string(w.data.size()) + " bytes, need " + std::to_string(need) + ")";
        return false;
      }
      if (!op.bias.empty()) {
        auto bit = g.weights.find(op.bias);
        if (bit == g.weights.end()) {
          error = "expected initializer '" + op.bias + "' was not found";
          return false;
        }
        const Weight& b = bit->second;
        if (b.dims.size() != 1 || b.dims[0] != w.dims[0]) {
          error = "Conv bias '" + op.bias +
                  "' must be a rank-1 tensor with the weight's channel count";
          return false;
        }
        if (b.dtype != onnx::kFloat && b.dtype != onnx::kFloat16) {
          error = "Conv bias '" + op.bias + "' has unsupported dtype " + std::to_string(b.dtype);
          return false;
        }
        if (b.data.size() < static_cast<size_t>(b.dims[0]) * onnx::DtypeSize(b.dtype)) {
          error = "Conv bias '" + op.bias + "' storage is truncated";
          return false;
        }
      }
    } else if (n.op_type == "Sigmoid" || n.op_type == "Relu") {
      op.kind = n.op_type == "Relu" ? OpKind::Relu : OpKind::Sigmoid;
      op.in0 = in(0);
    } else if (n.op_type == "Mul" || n.op_type == "Add") {
      op.kind = n.op_type == "Mul" ? OpKind::Mul : OpKind::Add;
      op.in0 = in(0);
      op.in1 = in(1);
    } else if (n.op_type == "Clip") {
      op.kind = OpKind::Clip;
      op.in0 = in(0);
      op.clip = true;
      if (auto a = n.attr("min")) op.clip_lo = a->f;
      if (auto a = n.attr("max")) op.clip_hi = a->f;
      if (!clip_scalar(in(1), op.clip_lo) || !clip_scalar(in(2), op.clip_hi)) return false;
    } else if (n.op_type == "DepthToSpace") {
      op.kind = OpKind::DepthToSpace;
      op.in0 = in(0);
      if (auto a = n.attr("blocksize")) op.blocksize = static_cast<int>(a->i);
      if (op.blocksize < 1) {
        error = "DepthToSpace blocksize must be positive";
        return false;
      }
      if (auto a = n.attr("mode"); a && a->s != "DCR") {
        error = "only DepthToSpace mode DCR is supported";
        return false;
      }
    } else {
      error = "unsupported op '" + n.op_type + "' in fused graph";
      return false;
    }
    g.ops.push_back(std::move(op));
  }

  // ---- fusion passes over the op list
  // A fusion renames the producing op's output to the consumer's output, so it
  // is legal only when the intermediate has exactly the consumers being fused
  // and is not the tensor the engine downloads.
  auto readers = [&](const std::string& t) {
    std::vector<size_t> r;
    for (size_t j = 0; j < g.ops.size(); ++j) {
      const Op& o = g.ops[j];
      bool uses = o.in0 == t || o.in1 == t;
      for (const auto& s : o.skips) uses = uses || s == t;
      if (uses) r.push_back(j);
    }
    return r;
  };
  auto protected_tensor = [&](const std::string& t) {
    if (t == g.output_name) return true;
    for (const auto& vi : og.outputs)
      if (vi.name == t) return true;
    return false;
  };
  auto erase = [&](std::vector<size_t> idx) {
    std::sort(idx.rbegin(), idx.rend());
    for (size_t i : idx) g.ops.erase(g.ops.begin() + static_cast<std::ptrdiff_t>(i));
  };
  auto producer_of = [&](const std::string& t) -> int {
    for (size_t j = 0; j < g.ops.size(); ++j)
      if (g.ops[j].out == t) return static_cast<int>(j);
    return -1;
  };

  bool changed = true;
  while (changed) {
    changed = false;
    for (size_t i = 0; i < g.ops.size() && !changed; ++i) {
      Op& c = g.ops[i];
      if (c.kind != OpKind::Conv || c.dts_b != 0) continue;
      const std::string co = c.out;
      if (protected_tensor(co)) continue;
      const auto rd = readers(co);
      const bool plain = c.act == kActNone && c.skips.empty() && !c.clip;
      // SiLU: x * Sigmoid(x) (hip_engine.cc:493-522).
      if (plain && rd.size() == 2) {
        size_t si = rd[0], mi = rd[1];
        if (g.ops[si].kind != OpKind::Sigmoid) std::swap(si, mi);
        const Op& s = g.ops[si];
        const Op& m = g.ops[mi];
        if (s.kind == OpKind::Sigmoid && s.in0 == co && m.kind == OpKind::Mul &&
            ((m.in0 == co && m.in1 == s.out) || (m.in1 == co && m.in0 == s.out)) &&
            !protected_tensor(s.out)) {
          const auto rs = readers(s.out);
          if (rs.size() == 1 && rs[0] == mi) {
            c.act = kActSilu;
            c.out = m.out;
            erase({si, mi});
            changed = true;
            continue;
          }
        }
      }
      if (rd.size() != 1) continue;
      Op& nx = g.ops[rd[0]];
      // ReLU.
      if (plain && nx.kind == OpKind::Relu) {
        c.act = kActRelu;
        c.out = nx.out;
        erase({rd[0]});
        changed = true;
        continue;
      }
      // Residual add: the conv output plus an activation that exists before the
      // conv runs (graph input or an earlier op). x + x is left alone: it would
      // bind the conv's own output as the residual.
      if (nx.kind == OpKind::Add && !c.clip && c.skips.size() < 2 && nx.in0 != nx.in1) {
        const std::string other = nx.in0 == co ? nx.in1 : nx.in0;
        const int p = producer_of(other);
        const bool early = other == g.input_name || (p >= 0 && p < static_cast<int>(i));
        if (early && !g.weights.count(other)) {
          c.skips.push_back(other);
          c.out = nx.out;
          erase({rd[0]});
          changed = true;
          continue;
        }
      }
      // Clip.
      if (nx.kind == OpKind::Clip && !c.clip) {
        c.clip = true;
        c.clip_lo = nx.clip_lo;
        c.clip_hi = nx.clip_hi;
        c.out = nx.out;
        erase({rd[0]});
        changed = true;
        continue;
      }
    }
    // DepthToSpace followed by its only consumer, a Clip (hip_engine.cc:543-570).
    for (size_t i = 0; i < g.ops.size() && !changed; ++i) {
      Op& d = g.ops[i];
      if (d.kind != OpKind::DepthToSpace || d.clip || protected_tensor(d.out)) continue;
      const auto rd = readers(d.out);
      if (rd.size() != 1 || g.ops[rd[0]].kind != OpKind::Clip) continue;
      d.clip = true;
      d.clip_lo = g.ops[rd[0]].clip_lo;
      d.clip_hi = g.ops[rd[0]].clip_hi;
      d.out = g.ops[rd[0]].out;
      erase({rd[0]});
      changed = true;
    }
    // Tail: a conv whose only consumer is a DepthToSpace producing the graph
    // output writes that output directly (clip commutes with the permutation).
    for (size_t i = 0; i < g.ops.size() && !changed; ++i) {
      Op& c = g.ops[i];
      if (c.kind != OpKind::Conv || c.dts_b != 0 || protected_tensor(c.out)) continue;
      const auto rd = readers(c.out);
      if (rd.size() != 1) continue;
      const Op& d = g.ops[rd[0]];
      if (d.kind != OpKind::DepthToSpace || d.out != g.output_name) continue;
      if (d.clip && c.clip) continue;
      c.dts_b = d.blocksize;
      if (d.clip) {
        c.clip = true;
        c.clip_lo = d.clip_lo;
        c.clip_hi = d.clip_hi;
      }
      c.out = d.out;
      erase({rd[0]});
      changed = true;
    }
  }

  // ---- operand validation: binary / unary operands and residual inputs must
  // be activations (hip_engine.cc:623-652).
  std::unordered_set<std::string> produced{g.input_name};
  for (const Op& op : g.ops) produced.insert(op.out);
  auto need = [&](const char* what, const std::string& t) {
    if (produced.count(t)) return true;
    error = std::string(what) + " operand '" + t +
            "' is not an activation produced in this graph; initializer constants and "
            "broadcasting are not supported";
    return false;
  };
  for (const Op& op : g.ops) {
    switch (op.kind) {
      case OpKind::Conv:
        if (!need("Conv input", op.in0)) return false;
        for (const auto& s : op.skips)
          if (!need("fused residual Add", s)) return false;
        break;
      case OpKind::Add:
      case OpKind::Mul:
        if (!need(OpKindName(op.kind), op.in0) || !need(OpKindName(op.kind), op.in1)) return false;
        break;
      default:
        if (!need("unary op", op.in0)) return false;
        break;
    }
  }
  if (!produced.count(g.output_name)) {
    error = "graph output '" + g.output_name + "' is not produced by any supported op";
    return false;
  }
  return true;
}

bool PropagateShapes(const Graph& g, const int64_t in[4],
                     std::unordered_map<std::string, Shape>& shapes) {
  shapes.clear();
  if (in[0] < 1 || in[1] < 1 || in[2] < 1 || in[3] < 1) return false;
  shapes[g.input_name] = Shape{in[0], in[2], in[3], in[1]};
  for (const Op& op : g.ops) {
    auto it = shapes.find(op.in0);
    if (it == shapes.end()) return false;
    const Shape s = it->second;
    Shape o = s;
    switch (op.kind) {
      case OpKind::Conv: {
        const Weight& w = g.weights.at(op.weight);
        if (w.dims[1] != s.c) return false;  // channel agreement
        o.c = w.dims[0];
        for (const auto& sk : op.skips) {
          auto k = shapes.find(sk);
          if (k == shapes.end() || k->second != o) return false;
        }
        if (op.dts_b >= 1) {
          const int64_t b = op.dts_b;
          if (o.c % (b * b) != 0) return false;
          o = Shape{o.n, o.h * b, o.w * b, o.c / (b * b)};
        }
        break;
      }
      case OpKind::Add:
      case OpKind::Mul: {
        auto k = shapes.find(op.in1);
        if (k == shapes.end() || k->second != s) return false;  // no broadcasting
        break;
      }
      case OpKind::DepthToSpace: {
        const int64_t b = op.blocksize;
        if (b < 1 || s.c % (b * b) != 0) return false;
        o = Shape{s.n, s.h * b, s.w * b, s.c / (b * b)};
        break;
      }
      default:
        break;
    }
    shapes[op.out] = o;
  }
  return shapes.count(g.output_name) != 0;
}

}  // namespace arthip
