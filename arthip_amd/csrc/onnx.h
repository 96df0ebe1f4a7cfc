// Minimal ONNX model reader: decodes the protobuf wire format of the
// ModelProto subset an ArtCNN-style conv chain uses (graph, nodes,
// attributes, initializers, value infos). The reference links libonnx /
// libprotobuf for this (src/vapoursynth/onnx_utils.cpp:95-128); this build has
// no protobuf dependency, so it decodes the wire format directly, with field
// numbers from the public onnx.proto.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace arthip {
namespace onnx {

// TensorProto.DataType values used here.
enum DataType : int32_t {
  kUndefined = 0,
  kFloat = 1,
  kUint8 = 2,
  kInt8 = 3,
  kUint16 = 4,
  kInt16 = 5,
  kInt32 = 6,
  kInt64 = 7,
  kString = 8,
  kBool = 9,
  kFloat16 = 10,
  kDouble = 11,
  kUint32 = 12,
  kUint64 = 13,
  kBfloat16 = 16,
};

struct Tensor {
  std::string name;
  std::vector<int64_t> dims;
  int32_t data_type = 0;
  std::string raw_data;
  std::vector<float> float_data;
  std::vector<int32_t> int32_data;
  std::vector<int64_t> int64_data;
  std::vector<double> double_data;
  int32_t data_location = 0;  // 1 = EXTERNAL
  bool has_external_data = false;
};

struct Attribute {
  std::string name;
  int32_t type = 0;  // AttributeProto.AttributeType
  float f = 0.0f;
  int64_t i = 0;
  std::string s;
  bool has_f = false, has_i = false, has_s = false, has_t = false;
  Tensor t;
  std::vector<float> floats;
  std::vector<int64_t> ints;
  std::vector<std::string> strings;
};

struct Node {
  std::vector<std::string> inputs;
  std::vector<std::string> outputs;
  std::string name;
  std::string op_type;
  std::string domain;
  std::vector<Attribute> attributes;

  const Attribute* attr(const std::string& n) const {
    for (const auto& a : attributes)
      if (a.name == n) return &a;
    return nullptr;
  }
};

struct ValueInfo {
  std::string name;
  int32_t elem_type = 0;
  bool has_shape = false;
  std::vector<int64_t> dims;  // -1 for symbolic / unknown
};

struct Graph {
  std::string name;
  std::vector<Node> nodes;
  std::vector<Tensor> initializers;
  std::vector<ValueInfo> inputs;
  std::vector<ValueInfo> outputs;
};

struct OpsetId {
  std::string domain;
  int64_t version = 0;
};

struct Model {
  int64_t ir_version = 0;
  std::vector<OpsetId> opset_import;
  std::string producer_name;
  Graph graph;
};

// Decodes a serialized ModelProto. Returns false (with a message) on malformed
// input; unknown fields are skipped as the protobuf rules require.
bool ParseModel(const void* data, size_t size, Model& model, std::string& error);
bool LoadModelFile(const std::string& path, Model& model, std::string& error);

// Element size in bytes for the dtypes the engine can materialise; 0 otherwise.
size_t DtypeSize(int32_t dtype);

}  // namespace onnx
}  // namespace arthip
