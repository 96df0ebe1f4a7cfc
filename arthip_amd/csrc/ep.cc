#include "ep.h"

#include <unordered_set>

#include "graph.h"

namespace arthip {

namespace {

using Inits = std::unordered_map<std::string, const onnx::Tensor*>;

Inits initializers(const onnx::Model& m) {
  Inits in;
  for (const auto& t : m.graph.initializers) in[t.name] = &t;
  return in;
}

int32_t type_of(const TypeMap& types, const std::string& name) {
  auto it = types.find(name);
  return it == types.end() ? onnx::kUndefined : it->second;
}

bool ints_are_one(const onnx::Attribute* a) {
  return a == nullptr || a->ints.size() < 2 || (a->ints[0] == 1 && a->ints[1] == 1);
}

// The run's external activations, constants and needed outputs
// (hip_execution_provider.cc:244-297), deduplicated in first-seen order.
void run_boundary(const onnx::Model& m, const Inits& inits,
                  const std::unordered_map<std::string, int>& total_consumers,
                  const std::unordered_set<std::string>& graph_outputs, const std::vector<int>& run,
                  std::vector<std::string>& acts, std::vector<std::string>& consts,
                  std::vector<std::string>& outs) {
  const auto& nodes = m.graph.nodes;
  std::unordered_set<std::string> produced;
  std::unordered_map<std::string, int> inside;
  for (int i : run) {
    for (const auto& o : nodes[i].outputs)
      if (!o.empty()) produced.insert(o);
    for (const auto& x : nodes[i].inputs)
      if (!x.empty()) ++inside[x];
  }
  std::unordered_set<std::string> seen_a, seen_c, seen_o;
  for (int i : run) {
    for (const auto& x : nodes[i].inputs) {
      if (x.empty() || produced.count(x)) continue;
      if (inits.count(x)) {
        if (seen_c.insert(x).second) consts.push_back(x);
      } else if (seen_a.insert(x).second) {
        acts.push_back(x);
      }
    }
    for (const auto& o : nodes[i].outputs) {
      if (o.empty()) continue;
      auto ti = total_consumers.find(o);
      auto ii = inside.find(o);
      const int total = ti == total_consumers.end() ? 0 : ti->second;
      const int in_run = ii == inside.end() ? 0 : ii->second;
      if ((total > in_run || graph_outputs.count(o)) && seen_o.insert(o).second) outs.push_back(o);
    }
  }
}

}  // namespace

TypeMap InferTypes(const onnx::Model& m) {
  TypeMap types;
  for (const auto& t : m.graph.initializers) types[t.name] = t.data_type;
  for (const auto& v : m.graph.inputs)
    if (!types.count(v.name)) types[v.name] = v.elem_type;
  for (const auto& n : m.graph.nodes) {
    int32_t t = onnx::kUndefined;
    if (n.op_type == "Cast") {
      const onnx::Attribute* to = n.attr("to");
      t = to ? static_cast<int32_t>(to->i) : onnx::kUndefined;
    } else if (!n.inputs.empty()) {
      t = type_of(types, n.inputs[0]);
    }
    for (const auto& o : n.outputs)
      if (!o.empty()) types[o] = t;
  }
  // Declared graph output types win where they are given.
  for (const auto& v : m.graph.outputs)
    if (v.elem_type != onnx::kUndefined) types[v.name] = v.elem_type;
  return types;
}

bool EpNodeSupported(const onnx::Model& m, const TypeMap& types, int i) {
  const onnx::Node& n = m.graph.nodes[i];
  const Inits inits = initializers(m);
  auto is_graph_input = [&](const std::string& name) {
    if (inits.count(name)) return false;
    for (const auto& v : m.graph.inputs)
      if (v.name == name) return true;
    return false;
  };
  auto is_graph_output = [&](const std::string& name) {
    for (const auto& v : m.graph.outputs)
      if (v.name == name) return true;
    return false;
  };

  // Boundary Casts fold into the IO conversion (hip_execution_provider.cc:25-53).
  if (n.op_type == "Cast") {
    if (n.inputs.empty() || n.outputs.empty() || n.inputs[0].empty() || n.outputs[0].empty())
      return false;
    const int32_t ti = type_of(types, n.inputs[0]), to = type_of(types, n.outputs[0]);
    if (ti == onnx::kFloat && to == onnx::kFloat16) return is_graph_input(n.inputs[0]);
    if (ti == onnx::kFloat16 && to == onnx::kFloat) return is_graph_output(n.outputs[0]);
    return false;
  }
  static const char* kOps[] = {"Conv", "Sigmoid", "Mul", "Add", "DepthToSpace", "Clip", "Relu"};
  bool known = false;
  for (const char* op : kOps) known = known || n.op_type == op;
  if (!known) return false;
  if (!n.domain.empty() && n.domain != "ai.onnx") return false;

  // fp16 tensors only (56-66), initializers included.
  for (const auto* defs : {&n.inputs, &n.outputs})
    for (const auto& x : *defs)
      if (!x.empty() && type_of(types, x) != onnx::kFloat16) return false;

  if (n.op_type == "Conv") {
    // Stride 1, dilation 1, group 1, symmetric 1-padding or SAME, 3x3 kernel
    // from an initializer (68-131).
    if (!ints_are_one(n.attr("strides")) || !ints_are_one(n.attr("dilations"))) return false;
    const onnx::Attribute* g = n.attr("group");
    if (g && g->i != 1) return false;
    bool pads_ok = false;
    if (const onnx::Attribute* p = n.attr("pads")) {
      if (p->ints.size() != 4) return false;
      for (int64_t v : p->ints)
        if (v != 1) return false;
      pads_ok = true;
    }
    if (const onnx::Attribute* ap = n.attr("auto_pad")) {
      if (ap->s == "SAME_UPPER" || ap->s == "SAME_LOWER")
        pads_ok = true;
      else if (ap->s != "NOTSET")
        return false;
    }
    if (!pads_ok || n.inputs.size() < 2) return false;
    auto w = inits.find(n.inputs[1]);
    if (w == inits.end()) return false;
    const auto& d = w->second->dims;
    if (d.size() != 4 || d[2] != 3 || d[3] != 3) return false;
    if (d[1] > MaxConvInputChannels() || d[0] > MaxConvOutputChannels()) return false;
  }
  if (n.op_type == "DepthToSpace") {
    const onnx::Attribute* mode = n.attr("mode");
    if (mode && mode->s != "DCR") return false;
    const onnx::Attribute* b = n.attr("blocksize");
    if (b && b->i < 1) return false;
  }
  if (n.op_type == "Clip") {
    // Input-form bounds must be initializers (146-159).
    for (size_t k = 1; k < n.inputs.size(); ++k)
      if (!n.inputs[k].empty() && !inits.count(n.inputs[k])) return false;
  }
  return true;
}

bool EpPartition(const onnx::Model& m, std::vector<EpRun>& runs, std::string& error) {
  runs.clear();
  const auto& nodes = m.graph.nodes;
  const Inits inits = initializers(m);
  // Topological order: every node input produced inside the graph is produced
  // by an earlier node.
  {
    std::unordered_set<std::string> producers, done;
    for (const auto& n : nodes)
      for (const auto& o : n.outputs)
        if (!o.empty()) producers.insert(o);
    for (const auto& n : nodes) {
      for (const auto& x : n.inputs)
        if (!x.empty() && producers.count(x) && !done.count(x)) {
          error = "model nodes are not in topological order (input '" + x + "' of node '" +
                  n.name + "')";
          return false;
        }
      for (const auto& o : n.outputs)
        if (!o.empty()) done.insert(o);
    }
  }
  const TypeMap types = InferTypes(m);

  // Maximal consecutive runs of supported nodes (204-221).
  std::vector<std::vector<int>> cand;
  std::vector<int> cur;
  for (int i = 0; i < static_cast<int>(nodes.size()); ++i) {
    if (EpNodeSupported(m, types, i)) {
      cur.push_back(i);
    } else if (!cur.empty()) {
      cand.push_back(cur);
      cur.clear();
    }
  }
  if (!cur.empty()) cand.push_back(cur);

  std::unordered_set<std::string> graph_outputs;
  for (const auto& v : m.graph.outputs) graph_outputs.insert(v.name);
  std::unordered_map<std::string, int> total_consumers;
  for (const auto& n : nodes)
    for (const auto& x : n.inputs)
      if (!x.empty()) ++total_consumers[x];

  for (const auto& run : cand) {
    std::vector<std::string> acts, consts, outs;
    run_boundary(m, inits, total_consumers, graph_outputs, run, acts, consts, outs);
    if (acts.size() != 1 || outs.size() != 1) continue;  // 298-302
    EpRun r;
    r.nodes = run;
    r.input = acts[0];
    r.constants = consts;
    r.output = outs[0];
    runs.push_back(std::move(r));
  }
  return true;
}

bool EpRunBoundary(const onnx::Model& m, const std::vector<int>& run,
                   std::vector<std::string>& acts, std::vector<std::string>& consts,
                   std::vector<std::string>& outs, std::string& error) {
  const auto& nodes = m.graph.nodes;
  acts.clear();
  consts.clear();
  outs.clear();
  if (run.empty()) {
    error = "empty node run";
    return false;
  }
  for (size_t k = 0; k < run.size(); ++k)
    if (run[k] < 0 || run[k] >= static_cast<int>(nodes.size()) || (k && run[k] <= run[k - 1])) {
      error = "node indices must be increasing and inside the graph";
      return false;
    }
  const Inits inits = initializers(m);
  std::unordered_set<std::string> graph_outputs;
  for (const auto& v : m.graph.outputs) graph_outputs.insert(v.name);
  std::unordered_map<std::string, int> total_consumers;
  for (const auto& n : nodes)
    for (const auto& x : n.inputs)
      if (!x.empty()) ++total_consumers[x];
  run_boundary(m, inits, total_consumers, graph_outputs, run, acts, consts, outs);
  return true;
}

bool EpNodeKeys(const onnx::Model& m, const std::vector<int>& nodes,
                std::vector<std::string>& keys, std::string& error) {
  keys.clear();
  for (int i : nodes) {
    if (i < 0 || i >= static_cast<int>(m.graph.nodes.size())) {
      error = "node index " + std::to_string(i) + " is outside the graph";
      return false;
    }
    const onnx::Node& n = m.graph.nodes[i];
    const std::string* key = nullptr;
    for (const auto& o : n.outputs)
      if (!o.empty()) {
        key = &o;
        break;
      }
    if (key == nullptr) {
      error = "node " + std::to_string(i) + " ('" + n.name + "', " + n.op_type +
              ") has no output to name it by";
      return false;
    }
    keys.push_back(*key);
  }
  return true;
}

bool EpRunModel(const onnx::Model& m, const std::vector<int>& run, onnx::Model& out,
                std::string& error) {
  const auto& nodes = m.graph.nodes;
  const Inits inits = initializers(m);
  std::vector<std::string> acts, consts, outs;
  if (!EpRunBoundary(m, run, acts, consts, outs, error)) return false;
  if (acts.size() != 1 || outs.size() != 1) {
    error = "a run needs exactly one activation input and one output (has " +
            std::to_string(acts.size()) + " and " + std::to_string(outs.size()) + ")";
    return false;
  }
  const TypeMap types = InferTypes(m);
  out = onnx::Model();
  out.ir_version = m.ir_version;
  out.opset_import = m.opset_import;
  out.producer_name = m.producer_name;
  out.graph.name = m.graph.name + "_run";
  for (int i : run) out.graph.nodes.push_back(nodes[i]);
  for (const auto& c : consts) out.graph.initializers.push_back(*inits.at(c));
  onnx::ValueInfo in;
  in.name = acts[0];
  in.elem_type = type_of(types, acts[0]);
  out.graph.inputs.push_back(in);
  onnx::ValueInfo o;
  o.name = outs[0];
  o.elem_type = type_of(types, outs[0]);
  out.graph.outputs.push_back(o);
  return true;
}

}  // namespace arthip
