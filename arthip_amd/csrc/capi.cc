// extern "C" surface of libarthip.so (include/arthip.h).
#include <hip/hip_runtime.h>

#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "arthip.h"
#include "clip.h"
#include "engine.h"
#include "ep.h"
#include "half.h"
#include "launch.h"
#include "pack.h"

static_assert(ARTHIP_DEBUG_POISON == arthip::kDebugPoison &&
                  ARTHIP_DEBUG_SYNC_EACH == arthip::kDebugSyncEach &&
                  ARTHIP_DEBUG_DUMP == arthip::kDebugDump &&
                  ARTHIP_DEBUG_UNFUSED == arthip::kDebugUnfused &&
                  ARTHIP_DEBUG_TRACE == arthip::kDebugTrace &&
                  ARTHIP_DEBUG_HOST_PROFILE == arthip::kDebugHostProfile &&
                  ARTHIP_DEBUG_DUMPOPS == arthip::kDebugDumpOps &&
                  ARTHIP_DEBUG_PLAN == arthip::kDebugPlan,
              "debug flag values of the C ABI and the engine differ");

struct arthip_engine {
  std::unique_ptr<arthip::Engine> eng;
};

struct arthip_vs_model {
  std::unique_ptr<arthip::ClipModel> m;
};

namespace {

thread_local std::string t_last_error;

int fail(const std::string& msg, int code) {
  t_last_error = msg;
  return code;
}

void copy_out(const std::string& s, char* dst, int len) {
  if (dst == nullptr || len <= 0) return;
  size_t n = s.size();
  if (n > static_cast<size_t>(len) - 1) n = static_cast<size_t>(len) - 1;
  std::memcpy(dst, s.data(), n);
  dst[n] = '\0';
}

int report(const std::string& msg, int code, char* err, int errlen) {
  t_last_error = msg;
  copy_out(msg, err, errlen);
  return code;
}

// C++ exceptions (allocation failure, a lookup that misses) must not unwind
// into the C caller: every entry point that can allocate runs its body through
// guard(), which turns them into that entry point's error return.
template <class F>
int guard(int code, char* err, int errlen, const char* prefix, F&& body) {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    return report(std::string(prefix) + "out of host memory", code, err, errlen);
  } catch (const std::exception& ex) {
    return report(std::string(prefix) + "internal error: " + ex.what(), code, err, errlen);
  } catch (...) {
    return report(std::string(prefix) + "internal error", code, err, errlen);
  }
}

constexpr int kMaxRank = 8;

void write_shape(const int64_t s[4], int64_t* out_shape, int* out_rank) {
  if (out_rank) *out_rank = 4;
  if (out_shape)
    for (int i = 0; i < 4 && i < kMaxRank; ++i) out_shape[i] = s[i];
}

// Fresh engine built from a model file (the test driver builds one per call,
// tests/correctness/harness/engine_harness.cc:63-145).
int make_engine(const char* path, int device, std::unique_ptr<arthip::Engine>& out,
                std::string& error) {
  if (path == nullptr) {
    error = "failed to parse model file (null path)";
    return ARTHIP_ERR_BUILD;
  }
  auto e = std::make_unique<arthip::Engine>(device);
  if (!e->BuildFile(path, error)) return ARTHIP_ERR_BUILD;
  if (!e->Init(error)) return ARTHIP_ERR_BUILD;
  out = std::move(e);
  return ARTHIP_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// Engine handle
// ---------------------------------------------------------------------------

int arthip_engine_create(int device_id, arthip_engine** out, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (out == nullptr) return report("null output handle", ARTHIP_ERR_BUILD, err, errlen);
    *out = nullptr;
    auto h = std::make_unique<arthip_engine>();
    h->eng = std::make_unique<arthip::Engine>(device_id);
    *out = h.release();
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

void arthip_engine_destroy(arthip_engine* eng) { delete eng; }

int arthip_engine_build_file(arthip_engine* eng, const char* path, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (eng == nullptr || path == nullptr)
      return report("null engine or path", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->BuildFile(path, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_build_bytes(arthip_engine* eng, const void* data, size_t size, char* err,
                              int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (eng == nullptr || data == nullptr)
      return report("null engine or model bytes", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->Build(data, size, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_output_shape(const arthip_engine* eng, const int64_t in_nchw[4],
                               int64_t out_nchw[4]) {
  return guard(ARTHIP_ERR_BUILD, nullptr, 0, "", [&]() -> int {
    if (eng == nullptr || in_nchw == nullptr || out_nchw == nullptr)
      return fail("null argument", ARTHIP_ERR_BUILD);
    if (!eng->eng->OutputShape(in_nchw, out_nchw)) return fail("shape propagation failed", ARTHIP_ERR_BUILD);
    return ARTHIP_OK;
  });
}

int arthip_engine_io_info(const arthip_engine* eng, int* in_fp32, int* out_fp32, int* in_channels,
                          int* out_channels) {
  if (eng == nullptr) return fail("null engine", ARTHIP_ERR_BUILD);
  if (in_fp32) *in_fp32 = eng->eng->InputFp32() ? 1 : 0;
  if (out_fp32) *out_fp32 = eng->eng->OutputFp32() ? 1 : 0;
  if (in_channels) *in_channels = eng->eng->InputChannels();
  if (out_channels) *out_channels = eng->eng->OutputChannels();
  return ARTHIP_OK;
}

int arthip_engine_run(arthip_engine* eng, const void* in_host, const int64_t in_nchw[4],
                      void* out_host, size_t out_cap, char* err, int errlen) {
  return guard(ARTHIP_ERR_RUN, err, errlen, "", [&]() -> int {
    if (eng == nullptr || in_nchw == nullptr)
      return report("null engine or shape", ARTHIP_ERR_BUILD, err, errlen);
    int64_t o[4];
    if (!eng->eng->OutputShape(in_nchw, o))
      return report("shape propagation failed", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->Run(in_host, in_nchw, out_host, out_cap, e))
      return report(e, ARTHIP_ERR_RUN, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_run_device(arthip_engine* eng, const void* in_dev, const int64_t in_nchw[4],
                             void* out_dev, void* stream, char* err, int errlen) {
  return guard(ARTHIP_ERR_RUN, err, errlen, "", [&]() -> int {
    if (eng == nullptr || in_nchw == nullptr)
      return report("null engine or shape", ARTHIP_ERR_BUILD, err, errlen);
    int64_t o[4];
    if (!eng->eng->OutputShape(in_nchw, o))
      return report("shape propagation failed", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->RunDevice(in_dev, in_nchw, out_dev, static_cast<hipStream_t>(stream), e))
      return report(e, ARTHIP_ERR_RUN, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_run_device_noalloc(arthip_engine* eng, const void* in_dev,
                                     const int64_t in_nchw[4], void* out_dev, void* stream,
                                     char* err, int errlen) {
  return guard(ARTHIP_ERR_RUN, err, errlen, "", [&]() -> int {
    if (eng == nullptr || in_nchw == nullptr)
      return report("null engine or shape", ARTHIP_ERR_BUILD, err, errlen);
    int64_t o[4];
    if (!eng->eng->OutputShape(in_nchw, o))
      return report("shape propagation failed", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->RunDeviceScratch(in_dev, in_nchw, out_dev, static_cast<hipStream_t>(stream),
                                    e))
      return report(e, ARTHIP_ERR_RUN, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_describe(const arthip_engine* eng, char* buf, int buflen) {
  return guard(ARTHIP_ERR_BUILD, nullptr, 0, "", [&]() -> int {
    if (eng == nullptr) return fail("null engine", ARTHIP_ERR_BUILD);
    copy_out(eng->eng->Describe(), buf, buflen);
    return ARTHIP_OK;
  });
}

int arthip_engine_set_profiling(arthip_engine* eng, int on) {
  if (eng == nullptr) return fail("null engine", ARTHIP_ERR_BUILD);
  eng->eng->SetProfiling(on != 0);
  return ARTHIP_OK;
}

int arthip_engine_set_debug(arthip_engine* eng, int flags, const char* dump_dir) {
  return guard(ARTHIP_ERR_BUILD, nullptr, 0, "", [&]() -> int {
    if (eng == nullptr) return fail("null engine", ARTHIP_ERR_BUILD);
    if ((flags & ~(ARTHIP_DEBUG_POISON | ARTHIP_DEBUG_SYNC_EACH | ARTHIP_DEBUG_DUMP |
                   ARTHIP_DEBUG_UNFUSED | ARTHIP_DEBUG_TRACE | ARTHIP_DEBUG_HOST_PROFILE |
                   ARTHIP_DEBUG_DUMPOPS | ARTHIP_DEBUG_PLAN)) != 0)
      return fail("unknown debug flag", ARTHIP_ERR_BUILD);
    if ((flags & ARTHIP_DEBUG_DUMP) && (dump_dir == nullptr || *dump_dir == '\0'))
      return fail("dump requested without a directory", ARTHIP_ERR_BUILD);
    eng->eng->SetDebug(flags, dump_dir ? dump_dir : "");
    return ARTHIP_OK;
  });
}

int arthip_engine_set_log(arthip_engine* eng, const char* path, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (eng == nullptr) return report("null engine", ARTHIP_ERR_BUILD, err, errlen);
    std::string e;
    if (!eng->eng->SetLog(path ? path : "", e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_get_debug(const arthip_engine* eng, int* flags) {
  if (eng == nullptr || flags == nullptr) return fail("null argument", ARTHIP_ERR_BUILD);
  *flags = eng->eng->DebugFlags();
  return ARTHIP_OK;
}

int arthip_engine_profile_read(arthip_engine* eng, int max_steps, double* total_ms,
                               int64_t* launches, char* names, int names_len, char* err,
                               int errlen) {
  return guard(-ARTHIP_ERR_RUN, err, errlen, "", [&]() -> int {
    if (eng == nullptr) return -report("null engine", ARTHIP_ERR_BUILD, err, errlen);
    std::vector<arthip::Engine::StepProfile> prof;
    std::string e;
    if (!eng->eng->ProfileRead(prof, e)) return -report(e, ARTHIP_ERR_RUN, err, errlen);
    std::string joined;
    const int n = static_cast<int>(prof.size());
    for (int i = 0; i < n; ++i) {
      if (i < max_steps) {
        if (total_ms) total_ms[i] = prof[i].total_ms;
        if (launches) launches[i] = prof[i].launches;
      }
      joined += prof[i].name;
      joined += '\n';
    }
    copy_out(joined, names, names_len);
    copy_out("", err, errlen);
    return n;
  });
}

// ---------------------------------------------------------------------------
// Test-driver ABI (engine_harness.cc:56-210)
// ---------------------------------------------------------------------------

int engine_device_count(int* count) {
  if (count == nullptr) return ARTHIP_ERR_BUILD;
  if (hipInit(0) != hipSuccess) return ARTHIP_ERR_BUILD;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return ARTHIP_ERR_BUILD;
  *count = n;
  return ARTHIP_OK;
}

int engine_probe(const char* model_path, int N, int H, int W, int C, int device, char* err,
                 int errlen, int* in_fp32, int* out_fp32, int* cin, int* cout,
                 int64_t* out_shape, int* out_rank) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    std::unique_ptr<arthip::Engine> eng;
    std::string e;
    if (make_engine(model_path, device, eng, e) != ARTHIP_OK) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    if (in_fp32) *in_fp32 = eng->InputFp32() ? 1 : 0;
    if (out_fp32) *out_fp32 = eng->OutputFp32() ? 1 : 0;
    if (cin) *cin = eng->InputChannels();
    if (cout) *cout = eng->OutputChannels();
    const int64_t in[4] = {N, C, H, W};
    int64_t o[4];
    if (!eng->OutputShape(in, o)) return report("shape propagation failed", ARTHIP_ERR_BUILD, err, errlen);
    write_shape(o, out_shape, out_rank);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int engine_run(const char* model_path, int N, int H, int W, int C, int device,
               const void* input, size_t input_bytes, void* out, size_t cap,
               size_t* out_bytes, int* out_fp32, int64_t* out_shape, int* out_rank, char* err,
               int errlen) {
  return guard(ARTHIP_ERR_RUN, err, errlen, "", [&]() -> int {
    std::unique_ptr<arthip::Engine> eng;
    std::string e;
    if (make_engine(model_path, device, eng, e) != ARTHIP_OK) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    const int64_t in[4] = {N, C, H, W};
    int64_t o[4];
    if (!eng->OutputShape(in, o)) return report("shape propagation failed", ARTHIP_ERR_BUILD, err, errlen);
    const size_t need = eng->OutputBytes(in);
    if (need > cap) return report("output buffer too small", ARTHIP_ERR_BUILD, err, errlen);
    const size_t expect = eng->InputBytes(in);
    if (input == nullptr || input_bytes != expect)
      return report("input buffer size mismatch (expected " + std::to_string(expect) +
                        " bytes, got " + std::to_string(input_bytes) + ")",
                    ARTHIP_ERR_BUILD, err, errlen);
    if (!eng->Run(input, in, out, cap, e)) return report(e, ARTHIP_ERR_RUN, err, errlen);
    if (out_bytes) *out_bytes = need;
    if (out_fp32) *out_fp32 = eng->OutputFp32() ? 1 : 0;
    write_shape(o, out_shape, out_rank);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int engine_alloc_failure_then_run(const char* model_path, int N, int bigH, int bigW, int C,
                                  int device, const void* recovery_input,
                                  size_t recovery_input_bytes, void* out, size_t cap,
                                  size_t* out_bytes, int* out_fp32, int64_t* out_shape,
                                  int* out_rank, char* failerr, int failerrlen, char* runerr,
                                  int runerrlen) {
  return guard(ARTHIP_ERR_RUN, runerr, runerrlen, "", [&]() -> int {
    std::unique_ptr<arthip::Engine> eng;
    std::string e;
    if (make_engine(model_path, device, eng, e) != ARTHIP_OK)
      return report("build failed: " + e, ARTHIP_ERR_BUILD, failerr, failerrlen);
    char dummy[8] = {0};
    const int64_t big[4] = {N, C, bigH, bigW};
    std::string first;
    if (eng->Run(dummy, big, dummy, sizeof(dummy), first))
      return report("expected the oversized run to fail but it succeeded", ARTHIP_ERR_BUILD, failerr,
                    failerrlen);
    copy_out(first, failerr, failerrlen);
    const int64_t in[4] = {N, C, 16, 16};
    int64_t o[4];
    if (!eng->OutputShape(in, o)) return report("recovery shape probe failed", ARTHIP_ERR_RUN, runerr, runerrlen);
    const size_t need = eng->OutputBytes(in);
    if (need > cap) return report("recovery output buffer too small", ARTHIP_ERR_RUN, runerr, runerrlen);
    if (recovery_input == nullptr || recovery_input_bytes != eng->InputBytes(in))
      return report("recovery input buffer size mismatch", ARTHIP_ERR_RUN, runerr, runerrlen);
    std::string second;
    if (!eng->Run(recovery_input, in, out, cap, second))
      return report(second, ARTHIP_ERR_RUN, runerr, runerrlen);
    if (out_bytes) *out_bytes = need;
    if (out_fp32) *out_fp32 = eng->OutputFp32() ? 1 : 0;
    write_shape(o, out_shape, out_rank);
    copy_out("", runerr, runerrlen);
    return ARTHIP_OK;
  });
}

// ---------------------------------------------------------------------------
// ONNX Runtime execution provider
// ---------------------------------------------------------------------------

int arthip_ep_get_capability(const void* model, size_t size, int device_id, int* n_runs,
                             int* run_start, int max_runs, int* n_nodes, int* nodes,
                             int max_nodes, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (n_runs) *n_runs = 0;
    if (n_nodes) *n_nodes = 0;
    if (model == nullptr || n_runs == nullptr || n_nodes == nullptr)
      return report("null model or output count", ARTHIP_ERR_BUILD, err, errlen);
    if (device_id >= 0) {
      // Context initialization (hip_execution_provider.cc:163-176): a device that
      // cannot be selected and initialized gets no nodes. The calling thread's
      // current device is restored afterwards.
      int prev = -1;
      const bool had = hipGetDevice(&prev) == hipSuccess;
      const bool ok = hipSetDevice(device_id) == hipSuccess && hipFree(nullptr) == hipSuccess;
      if (had) (void)hipSetDevice(prev);
      (void)hipGetLastError();
      if (!ok) {
        copy_out("", err, errlen);
        return ARTHIP_OK;
      }
    }
    arthip::onnx::Model m;
    std::string e;
    if (!arthip::onnx::ParseModel(model, size, m, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    std::vector<arthip::EpRun> runs;
    if (!arthip::EpPartition(m, runs, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    int total = 0;
    for (const auto& r : runs) total += static_cast<int>(r.nodes.size());
    *n_runs = static_cast<int>(runs.size());
    *n_nodes = total;
    if (static_cast<int>(runs.size()) + 1 > max_runs || total > max_nodes || run_start == nullptr ||
        (total > 0 && nodes == nullptr))
      return report("capability output arrays are too small", ARTHIP_ERR_BUILD, err, errlen);
    int k = 0;
    for (size_t r = 0; r < runs.size(); ++r) {
      run_start[r] = k;
      for (int i : runs[r].nodes) nodes[k++] = i;
    }
    run_start[runs.size()] = k;
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

// Writes names NUL-separated into (buf, len); false when they do not fit.
static bool pack_names(const std::vector<std::string>& names, char* buf, int len) {
  size_t need = 0;
  for (const auto& n : names) need += n.size() + 1;
  if (need > 0 && (buf == nullptr || need > static_cast<size_t>(len < 0 ? 0 : len))) return false;
  size_t k = 0;
  for (const auto& n : names) {
    std::memcpy(buf + k, n.data(), n.size());
    k += n.size();
    buf[k++] = '\0';
  }
  return true;
}

int arthip_ep_run_boundary(const void* model, size_t size, const int* nodes, int n_nodes,
                           char* activations, int activations_len, int* n_activations,
                           char* constants, int constants_len, int* n_constants, char* outputs,
                           int outputs_len, int* n_outputs, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (model == nullptr || (n_nodes > 0 && nodes == nullptr))
      return report("null model or node list", ARTHIP_ERR_BUILD, err, errlen);
    arthip::onnx::Model m;
    std::string e;
    if (!arthip::onnx::ParseModel(model, size, m, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    std::vector<std::string> acts, consts, outs;
    const std::vector<int> run(nodes, nodes + (n_nodes > 0 ? n_nodes : 0));
    if (!arthip::EpRunBoundary(m, run, acts, consts, outs, e))
      return report(e, ARTHIP_ERR_BUILD, err, errlen);
    if (n_activations) *n_activations = static_cast<int>(acts.size());
    if (n_constants) *n_constants = static_cast<int>(consts.size());
    if (n_outputs) *n_outputs = static_cast<int>(outs.size());
    if (!pack_names(acts, activations, activations_len) ||
        !pack_names(consts, constants, constants_len) || !pack_names(outs, outputs, outputs_len))
      return report("name buffers are too small", ARTHIP_ERR_BUILD, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_ep_node_keys(const void* model, size_t size, const int* nodes, int n_nodes,
                        char* keys, int keys_len, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (model == nullptr || (n_nodes > 0 && nodes == nullptr))
      return report("null model or node list", ARTHIP_ERR_BUILD, err, errlen);
    arthip::onnx::Model m;
    std::string e;
    if (!arthip::onnx::ParseModel(model, size, m, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    std::vector<std::string> names;
    const std::vector<int> run(nodes, nodes + (n_nodes > 0 ? n_nodes : 0));
    if (!arthip::EpNodeKeys(m, run, names, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    if (!pack_names(names, keys, keys_len))
      return report("key buffer is too small", ARTHIP_ERR_BUILD, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_engine_build_subgraph(arthip_engine* eng, const void* model, size_t size,
                                 const int* nodes, int n_nodes, char* err, int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    if (eng == nullptr || model == nullptr || (n_nodes > 0 && nodes == nullptr))
      return report("null engine, model or node list", ARTHIP_ERR_BUILD, err, errlen);
    arthip::onnx::Model m, sub;
    std::string e;
    if (!arthip::onnx::ParseModel(model, size, m, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    const std::vector<int> run(nodes, nodes + (n_nodes > 0 ? n_nodes : 0));
    if (!arthip::EpRunModel(m, run, sub, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    if (!eng->eng->BuildParsed(sub, e)) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

// ---------------------------------------------------------------------------
// VapourSynth filter core
// ---------------------------------------------------------------------------

static arthip::VideoFormat to_format(const arthip_vs_format& f) {
  arthip::VideoFormat v;
  v.color_family = f.color_family;
  v.sample_type = f.sample_type;
  v.bits_per_sample = f.bits_per_sample;
  v.sub_sampling_w = f.sub_sampling_w;
  v.sub_sampling_h = f.sub_sampling_h;
  v.num_planes = f.num_planes;
  return v;
}

int arthip_vs_model_create(const arthip_vs_model_args* args, int num_clips,
                           const arthip_vs_format* clip_format, int width, int height,
                           arthip_vs_model** out, arthip_vs_model_info* info, char* err,
                           int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "hip.Model: ", [&]() -> int {
    if (out == nullptr || args == nullptr || clip_format == nullptr)
      return report("hip.Model: null argument", ARTHIP_ERR_BUILD, err, errlen);
    *out = nullptr;
    arthip::ClipModelArgs a;
    if (args->network_size > 0 && args->network_data != nullptr) {
      const uint8_t* p = static_cast<const uint8_t*>(args->network_data);
      a.network_bytes.assign(p, p + args->network_size);
    } else if (args->network_path != nullptr) {
      a.network_path = args->network_path;
    } else {
      return report("hip.Model: network_path is required", ARTHIP_ERR_BUILD, err, errlen);
    }
    a.has_device_id = args->has_device_id != 0;
    a.device_id = args->device_id;
    a.has_num_streams = args->has_num_streams != 0;
    a.num_streams = args->num_streams;
    a.has_fp16 = args->has_fp16 != 0;
    a.fp16 = args->fp16;
    if (args->overlap && args->overlap_len > 0)
      a.overlap.assign(args->overlap, args->overlap + args->overlap_len);
    if (args->tilesize && args->tilesize_len > 0)
      a.tilesize.assign(args->tilesize, args->tilesize + args->tilesize_len);
    if (args->flexible_output_prop) a.flexible_output_prop = args->flexible_output_prop;
    std::string e;
    auto m = arthip::ClipModel::Create(a, num_clips, to_format(*clip_format), width, height, e);
    if (!m) return report(e, ARTHIP_ERR_BUILD, err, errlen);
    if (info) {
      const arthip::VideoFormat& f = m->out_format();
      info->format = arthip_vs_format{f.color_family, f.sample_type, f.bits_per_sample,
                                      f.sub_sampling_w, f.sub_sampling_h, f.num_planes};
      info->width = m->out_width();
      info->height = m->out_height();
      info->num_planes = m->out_channels();
      info->planes_written = m->planes_written();
      info->flexible = m->flexible() ? 1 : 0;
      info->in_fp32 = m->input_fp32() ? 1 : 0;
      info->out_fp32 = m->output_fp32() ? 1 : 0;
      info->num_streams = m->num_streams();
      info->scale_w = m->scale_w();
      info->scale_h = m->scale_h();
    }
    auto h = std::make_unique<arthip_vs_model>();
    h->m = std::move(m);
    *out = h.release();
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

int arthip_vs_model_get_frame(arthip_vs_model* model, const arthip_vs_format* fmt,
                              const int* plane_w, const int* plane_h, const void* const* src,
                              const ptrdiff_t* src_stride, void* const* dst,
                              const ptrdiff_t* dst_stride, int n_dst, char* err, int errlen) {
  return guard(ARTHIP_ERR_RUN, err, errlen, "hip.Model: ", [&]() -> int {
    if (model == nullptr || fmt == nullptr)
      return report("hip.Model: null model or format", ARTHIP_ERR_RUN, err, errlen);
    std::string e;
    if (!model->m->GetFrame(to_format(*fmt), plane_w, plane_h, src, src_stride, dst, dst_stride,
                            n_dst, e))
      return report(e, ARTHIP_ERR_RUN, err, errlen);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

void arthip_vs_model_destroy(arthip_vs_model* model) { delete model; }

int arthip_vs_version(char* version, int len, int* device_count) {
  copy_out(arthip_version(), version, len);
  if (device_count) {
    int n = 0;
    *device_count = hipGetDeviceCount(&n) == hipSuccess ? n : -1;
  }
  return ARTHIP_OK;
}

int arthip_vs_device_properties(int device_id, char* name, int namelen, int64_t* pci_device_id,
                                int64_t* clock_rate, int64_t* global_memory, char* err,
                                int errlen) {
  return guard(ARTHIP_ERR_BUILD, err, errlen, "", [&]() -> int {
    hipDeviceProp_t props{};
    if (hipGetDeviceProperties(&props, device_id) != hipSuccess)
      return report("hipDeviceProperties: failed to query device", ARTHIP_ERR_BUILD, err, errlen);
    copy_out(props.name, name, namelen);
    if (pci_device_id) *pci_device_id = props.pciDeviceID;
    if (clock_rate) *clock_rate = props.clockRate;
    if (global_memory) *global_memory = static_cast<int64_t>(props.totalGlobalMem);
    copy_out("", err, errlen);
    return ARTHIP_OK;
  });
}

// ---------------------------------------------------------------------------
// Kernel-level entry points
// ---------------------------------------------------------------------------

uint16_t arthip_f32_to_f16(float f) { return arthip::f32_to_f16(f); }
float arthip_f16_to_f32(uint16_t h) { return arthip::f16_to_f32(h); }
uint16_t arthip_f32_to_f16_no_subnormals(float f) { return arthip::f32_to_f16_no_subnormals(f); }
const char* arthip_last_error(void) { return t_last_error.c_str(); }
const char* arthip_version(void) { return "arthip-mi355x 0.1.0 (gfx950)"; }

int arthip_conv3x3_limits(int* max_c, int* max_m) {
  if (max_c) *max_c = 32 * arthip::winograd_max_kc();
  if (max_m) *max_m = arthip::winograd_max_m();
  return ARTHIP_OK;
}

int arthip_padded_dims(int H, int W, int* Hp, int* Wp) {
  if (H < 1 || W < 1) return fail("arthip_padded_dims: non-positive size", ARTHIP_ERR_BUILD);
  if (Hp) *Hp = static_cast<int>(arthip::padded_rows(H));
  if (Wp) *Wp = static_cast<int>(arthip::padded_cols(W));
  return ARTHIP_OK;
}

size_t arthip_conv3x3_packed_halfs(int M, int C) {
  if (M <= 0 || C <= 0) return 0;
  return C == 1 ? arthip::direct_packed_halfs(M) : arthip::winograd_packed_halfs(C, M);
}

size_t arthip_conv3x3_bias_len(int M) { return M <= 0 ? 0 : arthip::bias_padded_len(M); }

int arthip_conv3x3_pack(const uint16_t* w_oihw, const uint16_t* bias, int M, int C,
                        uint16_t* packed, size_t packed_cap, float* bias_out, size_t bias_cap) {
  return guard(ARTHIP_ERR_BUILD, nullptr, 0, "", [&]() -> int {
    if (w_oihw == nullptr || packed == nullptr || bias_out == nullptr || M <= 0 || C <= 0)
      return fail("arthip_conv3x3_pack: null buffer or non-positive channel count", ARTHIP_ERR_BUILD);
    if (C > 32 * arthip::winograd_max_kc() || M > arthip::winograd_max_m())
      return fail("arthip_conv3x3_pack: channel count beyond kernel limits", ARTHIP_ERR_BUILD);
    if (packed_cap < arthip_conv3x3_packed_halfs(M, C) || bias_cap < arthip_conv3x3_bias_len(M))
      return fail("arthip_conv3x3_pack: output buffer too small", ARTHIP_ERR_BUILD);
    std::vector<float> w(static_cast<size_t>(M) * C * 9);
    for (size_t i = 0; i < w.size(); ++i) w[i] = arthip::f16_to_f32(w_oihw[i]);
    std::vector<float> b(static_cast<size_t>(M), 0.0f);
    if (bias)
      for (int i = 0; i < M; ++i) b[i] = arthip::f16_to_f32(bias[i]);
    if (C == 1)
      arthip::direct_pack(w.data(), M, packed);
    else
      arthip::winograd_pack(w.data(), M, C, packed);
    arthip::bias_pad(b.data(), M, bias_out);
    return ARTHIP_OK;
  });
}

int arthip_conv3x3_f16_nhwc(const void* in, const void* packed, const float* bias, int act,
                            const void* skip0, const void* skip1, void* out, int N, int H, int W,
                            int C, int M, void* stream) {
  if (in == nullptr || packed == nullptr || bias == nullptr || out == nullptr)
    return fail("arthip_conv3x3_f16_nhwc: null buffer", ARTHIP_ERR_BUILD);
  if (N < 1 || H < 1 || W < 1 || C < 1 || M < 1)
    return fail("arthip_conv3x3_f16_nhwc: non-positive dimension", ARTHIP_ERR_BUILD);
  if (act < 0 || act > 2) return fail("arthip_conv3x3_f16_nhwc: unknown activation", ARTHIP_ERR_BUILD);
  if (C > 32 * arthip::winograd_max_kc() || M > arthip::winograd_max_m())
    return fail("arthip_conv3x3_f16_nhwc: channel count beyond kernel limits", ARTHIP_ERR_BUILD);
  arthip::Epilogue e{};
  e.bias = bias;
  e.skip0 = static_cast<const uint16_t*>(skip0);
  e.skip1 = static_cast<const uint16_t*>(skip1);
  e.out = out;
  e.act = act;
  e.out_kind = arthip::kOutPadded;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (C == 1) {
    arthip::DirectArgs a{};
    a.in = static_cast<const uint16_t*>(in);
    a.w = static_cast<const uint16_t*>(packed);
    a.epi = e;
    a.N = N; a.H = H; a.W = W; a.M = M;
    err = arthip::launch_direct(a, s);
  } else {
    arthip::WinoArgs a{};
    a.in = static_cast<const uint16_t*>(in);
    a.u = static_cast<const uint16_t*>(packed);
    a.epi = e;
    a.N = N; a.H = H; a.W = W; a.C = C; a.M = M;
    err = arthip::launch_winograd(a, s);
  }
  if (err != hipSuccess)
    return fail(std::string("conv3x3 launch failed: ") + hipGetErrorString(err), ARTHIP_ERR_RUN);
  return ARTHIP_OK;
}

int arthip_conv3x3_block_f16_nhwc(const void* in, const void* packed1, const float* bias1,
                                  int act1, const void* packed2, const float* bias2,
                                  const void* skip0, const void* skip1, void* out, int N, int H,
                                  int W, int C, void* stream) {
  if (in == nullptr || packed1 == nullptr || bias1 == nullptr || packed2 == nullptr ||
      bias2 == nullptr || out == nullptr)
    return fail("arthip_conv3x3_block_f16_nhwc: null buffer", ARTHIP_ERR_BUILD);
  if (skip0 == nullptr && skip1 != nullptr)
    return fail("arthip_conv3x3_block_f16_nhwc: skip1 without skip0", ARTHIP_ERR_BUILD);
  if (out == in || (skip0 != nullptr && out == skip0) || (skip1 != nullptr && out == skip1))
    return fail("arthip_conv3x3_block_f16_nhwc: out must not alias an input", ARTHIP_ERR_BUILD);
  if (act1 < 0 || act1 > 2)
    return fail("arthip_conv3x3_block_f16_nhwc: unknown activation", ARTHIP_ERR_BUILD);
  if (!arthip::block_eligible(C, C, act1, arthip::kActNone, N, H, W))
    return fail("arthip_conv3x3_block_f16_nhwc: the fused block needs C = 64, N, H, W >= 1 and "
                "a padded image below 2 GiB",
                ARTHIP_ERR_BUILD);
  arthip::BlockArgs a{};
  a.in = static_cast<const uint16_t*>(in);
  a.u1 = static_cast<const uint16_t*>(packed1);
  a.bias1 = bias1;
  a.u2 = static_cast<const uint16_t*>(packed2);
  a.bias2 = bias2;
  a.skip0 = static_cast<const uint16_t*>(skip0);
  a.skip1 = static_cast<const uint16_t*>(skip1);
  a.out = static_cast<uint16_t*>(out);
  a.N = N;
  a.H = H;
  a.W = W;
  a.act1 = act1;
  a.act2 = arthip::kActNone;
  const hipError_t err = arthip::launch_block(a, static_cast<hipStream_t>(stream));
  if (err != hipSuccess)
    return fail(std::string("conv3x3 block launch failed: ") + hipGetErrorString(err),
                ARTHIP_ERR_RUN);
  return ARTHIP_OK;
}

}  // extern "C"
