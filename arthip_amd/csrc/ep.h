// ONNX Runtime execution-provider partitioning: which nodes of a model the
// HIP EP claims, as maximal runs with one activation input and one output
// (src/onnxruntime-hip/hip_execution_provider.cc:22-177 IsNodeSupported,
// 181-335 GetCapability), and the model of one claimed run, which Compile hands
// to an engine (hip_execution_provider.cc:337-357 builds a HipGraph from the
// fused node's filtered graph instead).
//
// ORT supplies every tensor's type to IsNodeSupported; here the types come
// from a pass over the graph: graph inputs and initializers as declared, a
// Cast's output as its "to", every other op's outputs as its first input.
#pragma once

#include <string>
#include <unordered_map>
#include <vector>

#include "onnx.h"

namespace arthip {

using TypeMap = std::unordered_map<std::string, int32_t>;

struct EpRun {
  std::vector<int> nodes;              // indices into Graph::nodes, in graph order
  std::string input;                   // the run's one activation input
  std::vector<std::string> constants;  // initializers its nodes read
  std::string output;                  // the run's one exported output
};

TypeMap InferTypes(const onnx::Model& model);

// Whether node i would run on the EP. Two differences from the reference, both
// for models it cannot run: Relu is supported (the engine fuses it), and a Conv
// whose channel counts exceed the engine's limits is refused here instead of
// failing at compile time.
bool EpNodeSupported(const onnx::Model& model, const TypeMap& types, int i);

// GetCapability over a model whose nodes are in topological order (ONNX
// requires it; the order is checked). Runs with more than one activation input
// or more than one needed output are not claimed.
bool EpPartition(const onnx::Model& model, std::vector<EpRun>& runs, std::string& error);

// The boundary of a node run (any run, claimed or not): its external
// activations, the initializers it reads and the outputs needed outside it,
// each deduplicated in first-seen order (hip_execution_provider.cc:244-297).
bool EpRunBoundary(const onnx::Model& model, const std::vector<int>& nodes,
                   std::vector<std::string>& activations, std::vector<std::string>& constants,
                   std::vector<std::string>& outputs, std::string& error);

// The key of each listed node: its first non-empty output name. ONNX lets one
// node only produce a tensor name, so a key names one node of the graph in any
// serialization of it and in the caller's own node list, whatever their order
// and whatever nodes were added or removed elsewhere; node names may be empty
// or repeated and positions change with the order. Fails for an index outside
// the graph or a node without outputs.
bool EpNodeKeys(const onnx::Model& model, const std::vector<int>& nodes,
                std::vector<std::string>& keys, std::string& error);

// The model of one run: its nodes, the initializers they read, and the run's
// input and output as graph input and output with their inferred types.
bool EpRunModel(const onnx::Model& model, const std::vector<int>& nodes, onnx::Model& out,
                std::string& error);

}  // namespace arthip
