#include "onnx.h"

#include <cstdio>
#include <cstring>

namespace arthip {
namespace onnx {

namespace {

// Protobuf wire types.
enum Wire { kVarint = 0, kFixed64 = 1, kLen = 2, kFixed32 = 5 };

class Reader {
 public:
  Reader(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}

  bool done() const { return p_ >= end_; }
  bool ok() const { return ok_; }

  bool varint(uint64_t& v) {
    v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p_ >= end_) return fail();
      const uint8_t b = *p_++;
      v |= static_cast<uint64_t>(b & 0x7f) << shift;
      if ((b & 0x80) == 0) return true;
    }
    return fail();
  }

  bool key(uint32_t& field, uint32_t& wire) {
    uint64_t k;
    if (!varint(k)) return false;
    field = static_cast<uint32_t>(k >> 3);
    wire = static_cast<uint32_t>(k & 7);
    return field != 0 || fail();
  }

  bool bytes(const uint8_t*& b, size_t& n) {
    uint64_t len;
    if (!varint(len)) return false;
    if (len > static_cast<uint64_t>(end_ - p_)) return fail();
    b = p_;
    n = static_cast<size_t>(len);
    p_ += n;
    return true;
  }

  bool fixed32(uint32_t& v) {
    if (end_ - p_ < 4) return fail();
    std::memcpy(&v, p_, 4);
    p_ += 4;
    return true;
  }

  bool fixed64(uint64_t& v) {
    if (end_ - p_ < 8) return fail();
    std::memcpy(&v, p_, 8);
    p_ += 8;
    return true;
  }

  bool skip(uint32_t wire) {
    uint64_t v = 0;
    uint32_t v32;
    const uint8_t* b;
    size_t n;
    switch (wire) {
      case kVarint: return varint(v);
      case kFixed64: return fixed64(v);
      case kLen: return bytes(b, n);
      case kFixed32: return fixed32(v32);
      default: return fail();  // groups (3/4) are not used by onnx.proto
    }
  }

  bool string(std::string& s) {
    const uint8_t* b;
    size_t n;
    if (!bytes(b, n)) return false;
    s.assign(reinterpret_cast<const char*>(b), n);
    return true;
  }

  Reader sub(bool& okflag) {
    const uint8_t* b = nullptr;
    size_t n = 0;
    okflag = bytes(b, n);
    return Reader(b, n);
  }

  bool fail() {
    ok_ = false;
    return false;
  }

 private:
  const uint8_t* p_;
  const uint8_t* end_;
  bool ok_ = true;
};

// Repeated scalar fields may arrive packed (wire 2) or one value per key.
template <typename T>
bool ReadRepeatedVarint(Reader& r, uint32_t wire, std::vector<T>& out) {
  if (wire == kVarint) {
    uint64_t v = 0;
    if (!r.varint(v)) return false;
    out.push_back(static_cast<T>(static_cast<int64_t>(v)));
    return true;
  }
  if (wire != kLen) return r.fail();
  bool ok;
  Reader s = r.sub(ok);
  if (!ok) return false;
  while (!s.done()) {
    uint64_t v = 0;
    if (!s.varint(v)) return r.fail();
    out.push_back(static_cast<T>(static_cast<int64_t>(v)));
  }
  return true;
}

bool ReadRepeatedFloat(Reader& r, uint32_t wire, std::vector<float>& out) {
  auto put = [&](uint32_t bits) {
    float f;
    std::memcpy(&f, &bits, 4);
    out.push_back(f);
  };
  if (wire == kFixed32) {
    uint32_t v = 0;
    if (!r.fixed32(v)) return false;
    put(v);
    return true;
  }
  if (wire != kLen) return r.fail();
  bool ok;
  Reader s = r.sub(ok);
  if (!ok) return false;
  while (!s.done()) {
    uint32_t v = 0;
    if (!s.fixed32(v)) return r.fail();
    put(v);
  }
  return true;
}

bool ReadRepeatedDouble(Reader& r, uint32_t wire, std::vector<double>& out) {
  auto put = [&](uint64_t bits) {
    double d;
    std::memcpy(&d, &bits, 8);
    out.push_back(d);
  };
  if (wire == kFixed64) {
    uint64_t v = 0;
    if (!r.fixed64(v)) return false;
    put(v);
    return true;
  }
  if (wire != kLen) return r.fail();
  bool ok;
  Reader s = r.sub(ok);
  if (!ok) return false;
  while (!s.done()) {
    uint64_t v = 0;
    if (!s.fixed64(v)) return r.fail();
    put(v);
  }
  return true;
}

bool ParseTensor(Reader r, Tensor& t) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    switch (f) {
      case 1: ok = ReadRepeatedVarint(r, w, t.dims); break;
      case 2: {
        uint64_t v = 0;
        ok = w == kVarint && r.varint(v);
        t.data_type = static_cast<int32_t>(v);
        break;
      }
      case 4: ok = ReadRepeatedFloat(r, w, t.float_data); break;
      case 5: ok = ReadRepeatedVarint(r, w, t.int32_data); break;
      case 7: ok = ReadRepeatedVarint(r, w, t.int64_data); break;
      case 8: ok = w == kLen && r.string(t.name); break;
      case 9: ok = w == kLen && r.string(t.raw_data); break;
      case 10: ok = ReadRepeatedDouble(r, w, t.double_data); break;
      case 13:
        t.has_external_data = true;
        ok = r.skip(w);
        break;
      case 14: {
        uint64_t v = 0;
        ok = w == kVarint && r.varint(v);
        t.data_location = static_cast<int32_t>(v);
        break;
      }
      default: ok = r.skip(w); break;
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseAttribute(Reader r, Attribute& a) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    switch (f) {
      case 1: ok = w == kLen && r.string(a.name); break;
      case 20: {
        uint64_t v = 0;
        ok = w == kVarint && r.varint(v);
        a.type = static_cast<int32_t>(v);
        break;
      }
      case 2: {
        uint32_t v = 0;
        ok = w == kFixed32 && r.fixed32(v);
        std::memcpy(&a.f, &v, 4);
        a.has_f = true;
        break;
      }
      case 3: {
        uint64_t v = 0;
        ok = w == kVarint && r.varint(v);
        a.i = static_cast<int64_t>(v);
        a.has_i = true;
        break;
      }
      case 4:
        ok = w == kLen && r.string(a.s);
        a.has_s = true;
        break;
      case 5: {
        bool sok;
        Reader s = r.sub(sok);
        ok = w == kLen && sok && ParseTensor(s, a.t);
        a.has_t = true;
        break;
      }
      case 7: ok = ReadRepeatedFloat(r, w, a.floats); break;
      case 8: ok = ReadRepeatedVarint(r, w, a.ints); break;
      case 9: {
        std::string s;
        ok = w == kLen && r.string(s);
        a.strings.push_back(s);
        break;
      }
      default: ok = r.skip(w); break;
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseNode(Reader r, Node& n) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    std::string s;
    switch (f) {
      case 1:
        ok = w == kLen && r.string(s);
        n.inputs.push_back(s);
        break;
      case 2:
        ok = w == kLen && r.string(s);
        n.outputs.push_back(s);
        break;
      case 3: ok = w == kLen && r.string(n.name); break;
      case 4: ok = w == kLen && r.string(n.op_type); break;
      case 7: ok = w == kLen && r.string(n.domain); break;
      case 5: {
        bool sok;
        Reader sub = r.sub(sok);
        Attribute a;
        ok = w == kLen && sok && ParseAttribute(sub, a);
        n.attributes.push_back(std::move(a));
        break;
      }
      default: ok = r.skip(w); break;
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseDim(Reader r, int64_t& dim) {
  dim = -1;
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kVarint) {
      uint64_t v = 0;
      ok = r.varint(v);
      dim = static_cast<int64_t>(v);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseShape(Reader r, ValueInfo& vi) {
  vi.has_shape = true;
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kLen) {
      bool sok;
      Reader s = r.sub(sok);
      int64_t d;
      ok = sok && ParseDim(s, d);
      vi.dims.push_back(d);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseTensorType(Reader r, ValueInfo& vi) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kVarint) {
      uint64_t v = 0;
      ok = r.varint(v);
      vi.elem_type = static_cast<int32_t>(v);
    } else if (f == 2 && w == kLen) {
      bool sok;
      Reader s = r.sub(sok);
      ok = sok && ParseShape(s, vi);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseType(Reader r, ValueInfo& vi) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kLen) {
      bool sok;
      Reader s = r.sub(sok);
      ok = sok && ParseTensorType(s, vi);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseValueInfo(Reader r, ValueInfo& vi) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kLen) {
      ok = r.string(vi.name);
    } else if (f == 2 && w == kLen) {
      bool sok;
      Reader s = r.sub(sok);
      ok = sok && ParseType(s, vi);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseGraph(Reader r, Graph& g) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    bool sok = true;
    switch (f) {
      case 1: {
        Reader s = r.sub(sok);
        Node n;
        ok = w == kLen && sok && ParseNode(s, n);
        g.nodes.push_back(std::move(n));
        break;
      }
      case 2: ok = w == kLen && r.string(g.name); break;
      case 5: {
        Reader s = r.sub(sok);
        Tensor t;
        ok = w == kLen && sok && ParseTensor(s, t);
        g.initializers.push_back(std::move(t));
        break;
      }
      case 11:
      case 12: {
        Reader s = r.sub(sok);
        ValueInfo vi;
        ok = w == kLen && sok && ParseValueInfo(s, vi);
        (f == 11 ? g.inputs : g.outputs).push_back(std::move(vi));
        break;
      }
      default: ok = r.skip(w); break;
    }
    if (!ok) return false;
  }
  return r.ok();
}

bool ParseOpset(Reader r, OpsetId& o) {
  uint32_t f, w;
  while (!r.done()) {
    if (!r.key(f, w)) return false;
    bool ok = true;
    if (f == 1 && w == kLen) {
      ok = r.string(o.domain);
    } else if (f == 2 && w == kVarint) {
      uint64_t v = 0;
      ok = r.varint(v);
      o.version = static_cast<int64_t>(v);
    } else {
      ok = r.skip(w);
    }
    if (!ok) return false;
  }
  return r.ok();
}

}  // namespace

size_t DtypeSize(int32_t dtype) {
  switch (dtype) {
    case kFloat: case kInt32: case kUint32: return 4;
    case kFloat16: case kBfloat16: case kInt16: case kUint16: return 2;
    case kDouble: case kInt64: case kUint64: return 8;
    case kUint8: case kInt8: case kBool: return 1;
    default: return 0;
  }
}

bool ParseModel(const void* data, size_t size, Model& model, std::string& error) {
  model = Model();
  Reader r(static_cast<const uint8_t*>(data), size);
  uint32_t f, w;
  bool have_graph = false;
  while (!r.done()) {
    if (!r.key(f, w)) break;
    bool ok = true;
    bool sok = true;
    switch (f) {
      case 1: {
        uint64_t v = 0;
        ok = w == kVarint && r.varint(v);
        model.ir_version = static_cast<int64_t>(v);
        break;
      }
      case 2: ok = w == kLen && r.string(model.producer_name); break;
      case 7: {
        Reader s = r.sub(sok);
        ok = w == kLen && sok && ParseGraph(s, model.graph);
        have_graph = true;
        break;
      }
      case 8: {
        Reader s = r.sub(sok);
        OpsetId o;
        ok = w == kLen && sok && ParseOpset(s, o);
        model.opset_import.push_back(o);
        break;
      }
      default: ok = r.skip(w); break;
    }
    if (!ok) break;
  }
  if (!r.ok()) {
    error = "failed to parse model file (malformed protobuf)";
    return false;
  }
  if (!have_graph) {
    error = "failed to parse model file (no graph)";
    return false;
  }
  return true;
}

bool LoadModelFile(const std::string& path, Model& model, std::string& error) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    error = "failed to parse model file (cannot open '" + path + "')";
    return false;
  }
  std::string buf;
  char chunk[1 << 16];
  size_t n;
  while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.append(chunk, n);
  std::fclose(f);
  return ParseModel(buf.data(), buf.size(), model, error);
}

}  // namespace onnx
}  // namespace arthip
