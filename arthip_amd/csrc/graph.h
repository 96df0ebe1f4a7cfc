// Graph IR for the conv-chain engine: an ONNX graph lowered to a short list of
// fused ops.
//
// Mirrors the reference's OpSpec / WeightSpec / TensorInfo
// (src/vapoursynth/hip_engine.h:19-83; src/onnxruntime-hip/hip_graph.h:19-89)
// and its Build / PropagateShapes semantics (hip_engine.cc:197-736), with the
// capabilities the benchmark configs need on top: fused ReLU, up to two
// residual inputs per conv, a conv that writes the final DepthToSpace (+Clip)
// output directly, batch N >= 1 and up to 128 output channels.
#pragma once

#include <cstdint>
#include <limits>
#include <string>
#include <unordered_map>
#include <vector>

#include "onnx.h"

namespace arthip {

enum class OpKind { Conv, Sigmoid, Relu, Mul, Add, Clip, DepthToSpace };

const char* OpKindName(OpKind k);

// A materialised initializer: raw little-endian bytes in the declared dtype.
struct Weight {
  std::vector<uint8_t> data;
  std::vector<int64_t> dims;
  int32_t dtype = 0;
};

struct Op {
  OpKind kind = OpKind::Conv;
  std::string in0;  // activation input
  std::string in1;  // second activation (Add / Mul)
  std::string out;

  // Conv
  std::string weight;
  std::string bias;                // empty: no bias
  int act = 0;                     // fused activation (Act in conv_args.h)
  std::vector<std::string> skips;  // fused residual inputs, in graph order (<= 2)
  int dts_b = 0;                   // >= 1: fused DepthToSpace writing the graph output

  // Clip (standalone, or fused into a Conv / DepthToSpace)
  bool clip = false;
  float clip_lo = -std::numeric_limits<float>::infinity();
  float clip_hi = std::numeric_limits<float>::infinity();

  // DepthToSpace
  int blocksize = 1;
};

struct Graph {
  std::string input_name;   // activation the engine uploads (after a folded Cast)
  std::string output_name;  // activation the engine downloads (before a folded Cast)
  bool input_fp32 = false;
  bool output_fp32 = false;
  std::vector<Op> ops;
  std::unordered_map<std::string, Weight> weights;
};

// NHWC activation shape.
struct Shape {
  int64_t n = 0, h = 0, w = 0, c = 0;
  bool operator==(const Shape& o) const { return n == o.n && h == o.h && w == o.w && c == o.c; }
  bool operator!=(const Shape& o) const { return !(*this == o); }
};

// Largest channel counts the conv kernels accept.
int MaxConvInputChannels();
int MaxConvOutputChannels();

// Load-time conversion of an fp32 model to fp16, as the VapourSynth filter
// applies it with fp16=1 (src/vapoursynth/vs_hip.cpp:503-515, through
// convert_float_to_float16 with force_fp16_initializers): fp32 initializers are
// rounded with the converter's rule (f32_to_f16_no_subnormals), and fp32 graph
// inputs / outputs become fp16 unless keep_io_fp32 keeps them behind boundary
// Casts (the converter's cast_input / cast_output).
struct BuildOptions {
  bool fp16 = false;
  bool keep_io_fp32 = false;
};

// Parses, validates and fuses. Error messages keep the reference's wording
// where its tests match on them (tests/correctness/test_engine.py).
bool BuildGraph(const onnx::Model& model, Graph& g, std::string& error,
                const BuildOptions& opts = BuildOptions());

// NCHW input shape -> NHWC shape of every activation. Fails on geometry the
// kernels cannot run (channel mismatch, residual/binary shape mismatch,
// DepthToSpace block size).
bool PropagateShapes(const Graph& g, const int64_t in_nchw[4],
                     std::unordered_map<std::string, Shape>& shapes);

// Weight element as float (fp32 or fp16 storage), hip_engine.cc:1234-1249.
float WeightAt(const Weight& w, size_t idx);

}  // namespace arthip
