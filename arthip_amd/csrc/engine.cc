#include "engine.h"

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "half.h"
#include "launch.h"
#include "pack.h"
#include "plan_rules.h"

namespace arthip {

namespace {

std::string HipErr(const char* what, hipError_t e) {
  return std::string(what) + " failed: " + hipGetErrorString(e);
}

size_t PaddedBytes(const Shape& s) {
  return static_cast<size_t>(s.n) * static_cast<size_t>(padded_rows(s.h)) *
         static_cast<size_t>(padded_cols(s.w)) * static_cast<size_t>(s.c) * 2;
}

}  // namespace

Engine::Engine(int device_id) : device_(device_id) {
  auto on = [](const char* name) {
    const char* e = std::getenv(name);
    return e != nullptr && *e == '1';
  };
  if (on("VSHIP_POISON")) debug_ |= kDebugPoison;
  if (on("VSHIP_SYNC_EACH")) debug_ |= kDebugSyncEach;
  if (const char* d = std::getenv("VSHIP_DUMP")) {
    if (*d != '\0') {
      debug_ |= kDebugDump;
      dump_dir_ = d;
    }
  }
  if (on("VSHIP_TRACE")) debug_ |= kDebugTrace;
  if (on("HIP_PROFILE")) debug_ |= kDebugHostProfile;
  if (std::getenv("HIP_DUMPOPS") != nullptr) debug_ |= kDebugDumpOps;  // set, any value
  if (on("VSHIP_DEBUG")) debug_ |= kDebugPlan;
}

Engine::~Engine() {
  FreeAll();
  for (const EventPair& ev : pending_events_) {
    hipEventDestroy(ev.start);
    hipEventDestroy(ev.stop);
  }
  for (hipEvent_t e : event_pool_) hipEventDestroy(e);
  if (stream_) {
    hipSetDevice(device_);
    hipStreamDestroy(stream_);
  }
  if (run_done_) hipEventDestroy(run_done_);
  if (log_) std::fclose(log_);
}

bool Engine::SetLog(const std::string& path, std::string& error) {
  std::lock_guard<std::mutex> lock(mu_);
  FILE* f = nullptr;
  if (!path.empty()) {
    f = std::fopen(path.c_str(), "a");
    if (f == nullptr) {
      error = "cannot open log file '" + path + "'";
      return false;
    }
  }
  if (log_) std::fclose(log_);
  log_ = f;
  return true;
}

void Engine::Log(const char* fmt, ...) {
  FILE* f = log_ ? log_ : stderr;
  va_list ap;
  va_start(ap, fmt);
  std::vfprintf(f, fmt, ap);
  va_end(ap);
  std::fflush(f);
}

// Trace and host-profile lines of one Run / RunDevice call (VSHIP_TRACE,
// hip_engine.cc:1280-1298,1421-1425,1619; HIP_PROFILE, hip_graph.cc:1213-1447).
// The destructor reports a call that returned without Done as failed, with
// the error text it left.
struct Engine::RunLog {
  using Clock = std::chrono::steady_clock;
  Engine& e;
  const std::string& error;
  const bool trace, prof, host;
  uint64_t no = 0;
  bool done = false;
  Clock::time_point t0 = Clock::now(), t_built, t_in, t_launched, t_back;

  RunLog(Engine& eng, const char* what, const void* in, bool host_io, const std::string& err)
      : e(eng), error(err), trace((eng.debug_ & kDebugTrace) != 0),
        prof((eng.debug_ & kDebugHostProfile) != 0), host(host_io) {
    if (trace) {
      no = ++e.run_no_;
      e.Log("[run] enter #%llu %s in=%p\n", (unsigned long long)no, what, in);
    }
  }
  void Built() {
    t_built = Clock::now();
    if (trace) e.Log("[run] built #%llu\n", (unsigned long long)no);
  }
  void Uploaded() { t_in = Clock::now(); }
  void Launched() { t_launched = Clock::now(); }
  void Back() { t_back = Clock::now(); }
  static double ms(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
  }
  bool Done(const void* out) {
    done = true;
    const Clock::time_point t_end = Clock::now();
    if (prof) {
      if (host) {
        e.Log("[hipprof] build=%.3fms memin=%.3fms launch=%.3fms readback+wait=%.3fms\n",
              ms(t0, t_built), ms(t_built, t_in), ms(t_in, t_launched), ms(t_launched, t_back));
        e.Log("[hipprof] memout=%.3fms total=%.3fms\n", ms(t_back, t_end), ms(t0, t_end));
      } else {
        e.Log("[hipprof] build=%.3fms launch=%.3fms total=%.3fms (device-resident, not waited "
              "for)\n", ms(t0, t_built), ms(t_built, t_launched), ms(t0, t_end));
      }
    }
    if (trace) e.Log("[run] done #%llu out=%p\n", (unsigned long long)no, out);
    return true;
  }
  ~RunLog() {
    if (trace && !done)
      e.Log("[run] fail #%llu: %s\n", (unsigned long long)no, error.c_str());
  }
};

std::string Engine::BufLabel(const Plan& p, int idx, const void* in_dev,
                             const void* out_dev) const {
  char buf[160];
  if (idx == kBoundaryIn)
    std::snprintf(buf, sizeof buf, "input(%p,%.2fMB)", in_dev, p.in_bytes / 1048576.0);
  else if (idx == kBoundaryOut)
    std::snprintf(buf, sizeof buf, "output(%p,%.2fMB)", out_dev, p.out_bytes / 1048576.0);
  else
    std::snprintf(buf, sizeof buf, "%d(%p,%.2fMB)", idx, p.bufs[idx].ptr,
                  p.bufs[idx].bytes / 1048576.0);
  return buf;
}

void Engine::SetDebug(int flags, const std::string& dump_dir) {
  std::lock_guard<std::mutex> lock(mu_);
  flags &= kDebugAll;
  if ((flags ^ debug_) & kDebugUnfused) {  // the plans depend on it
    FreePlan();
    ClearPlan(scratch_plan_);
  }
  debug_ = flags;
  dump_dir_ = dump_dir;
  dump_runs_ = 0;
}

int Engine::DebugFlags() const {
  std::lock_guard<std::mutex> lock(mu_);
  return debug_;
}

// The previous run may still be executing on another stream; this run reuses
// its activation buffers, so its first launch waits for that run's event.
bool Engine::WaitPrevious(hipStream_t s, std::string& error) {
  if (last_stream_ == nullptr || last_stream_ == s) return true;
  const hipError_t e = hipStreamWaitEvent(s, run_done_, 0);
  if (e != hipSuccess) {
    error = HipErr("hipStreamWaitEvent on the previous run", e);
    return false;
  }
  return true;
}

// For a run captured into a HIP graph: its nodes cannot wait on an event
// recorded outside the capture, so the previous run must already be over.
bool Engine::PreviousDone(std::string& error) {
  if (last_stream_ == nullptr) return true;
  const hipError_t e = hipEventQuery(run_done_);
  if (e == hipSuccess) {
    last_stream_ = nullptr;
    return true;
  }
  error = e == hipErrorNotReady
              ? "the previous run on this handle is still executing; a run captured into a HIP "
                "graph cannot wait for it (synchronize before capturing)"
              : HipErr("hipEventQuery of the previous run", e);
  return false;
}

static bool StreamCapturing(hipStream_t s, bool& capturing, std::string& error) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess) {
    error = HipErr("hipStreamIsCapturing", e);
    return false;
  }
  capturing = cs != hipStreamCaptureStatusNone;
  return true;
}

// Blocks until the last enqueued run has finished (before its buffers are
// freed or replaced).
bool Engine::DrainPrevious() {
  if (last_stream_ == nullptr) return true;
  const hipError_t e = hipEventSynchronize(run_done_);
  last_stream_ = nullptr;
  return e == hipSuccess;
}

bool Engine::SetDevice(std::string& error) const {
  const hipError_t e = hipSetDevice(device_);
  if (e != hipSuccess) {
    error = "hipSetDevice(" + std::to_string(device_) + ") failed: " + hipGetErrorString(e);
    return false;
  }
  return true;
}

bool Engine::Init(std::string& error) {
  if (stream_ != nullptr) return SetDevice(error);
  const hipError_t ie = hipInit(0);
  if (ie != hipSuccess) {
    error = HipErr("hipInit", ie);
    return false;
  }
  if (!SetDevice(error)) return false;
  if (run_done_ == nullptr) {
    const hipError_t e = hipEventCreateWithFlags(&run_done_, hipEventDisableTiming);
    if (e != hipSuccess) {
      run_done_ = nullptr;
      error = HipErr("hipEventCreate", e);
      return false;
    }
  }
  const hipError_t e = hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking);
  if (e != hipSuccess) {
    stream_ = nullptr;
    error = HipErr("hipStreamCreate", e);
    return false;
  }
  // Set-up of the no-allocation entry point's scratch on this device (its
  // address resolved and its ordering event created once per device, here
  // with the device current), so that entry point's own calls create
  // nothing. A failure is reported by that entry point.
  std::string ignored;
  (void)scratch_setup(device_, ignored);
  return true;
}

bool Engine::Build(const void* data, size_t size, std::string& error, const BuildOptions& opts) {
  std::lock_guard<std::mutex> lock(mu_);
  onnx::Model model;
  if (!onnx::ParseModel(data, size, model, error)) return false;
  FreeAll();
  built_ = false;
  if (!BuildGraph(model, graph_, error, opts)) return false;
  built_ = true;
  return true;
}

bool Engine::BuildFile(const std::string& path, std::string& error, const BuildOptions& opts) {
  std::lock_guard<std::mutex> lock(mu_);
  onnx::Model model;
  if (!onnx::LoadModelFile(path, model, error)) return false;
  FreeAll();
  built_ = false;
  if (!BuildGraph(model, graph_, error, opts)) return false;
  built_ = true;
  return true;
}

bool Engine::BuildParsed(const onnx::Model& model, std::string& error, const BuildOptions& opts) {
  std::lock_guard<std::mutex> lock(mu_);
  FreeAll();
  built_ = false;
  if (!BuildGraph(model, graph_, error, opts)) return false;
  built_ = true;
  return true;
}

bool Engine::InputFp32() const {
  std::lock_guard<std::mutex> lock(mu_);
  return graph_.input_fp32;
}

bool Engine::OutputFp32() const {
  std::lock_guard<std::mutex> lock(mu_);
  return graph_.output_fp32;
}

int Engine::InputChannels() const {
  std::lock_guard<std::mutex> lock(mu_);
  for (const Op& op : graph_.ops)
    if (op.kind == OpKind::Conv) return static_cast<int>(graph_.weights.at(op.weight).dims[1]);
  return 1;
}

int Engine::OutputChannels() const {
  std::lock_guard<std::mutex> lock(mu_);
  for (auto it = graph_.ops.rbegin(); it != graph_.ops.rend(); ++it)
    if (it->kind == OpKind::Conv) return static_cast<int>(graph_.weights.at(it->weight).dims[0]);
  return 1;
}

bool Engine::OutputShape(const int64_t in[4], int64_t out[4]) const {
  std::lock_guard<std::mutex> lock(mu_);
  return OutputShapeUnlocked(in, out);
}

bool Engine::OutputShapeUnlocked(const int64_t in[4], int64_t out[4]) const {
  if (!built_) return false;
  std::unordered_map<std::string, Shape> shapes;
  if (!PropagateShapes(graph_, in, shapes)) return false;
  const Shape& s = shapes.at(graph_.output_name);
  out[0] = s.n;
  out[1] = s.c;
  out[2] = s.h;
  out[3] = s.w;
  return true;
}

size_t Engine::InputBytes(const int64_t in[4]) const {
  std::lock_guard<std::mutex> lock(mu_);
  return static_cast<size_t>(in[0] * in[1] * in[2] * in[3]) * (graph_.input_fp32 ? 4 : 2);
}

size_t Engine::OutputBytes(const int64_t in[4]) const {
  std::lock_guard<std::mutex> lock(mu_);
  return OutputBytesUnlocked(in);
}

size_t Engine::OutputBytesUnlocked(const int64_t in[4]) const {
  int64_t o[4];
  if (!OutputShapeUnlocked(in, o)) return 0;
  return static_cast<size_t>(o[0] * o[1] * o[2] * o[3]) * (graph_.output_fp32 ? 4 : 2);
}

void Engine::ClearPlan(Plan& p) {
  const bool scratch = p.scratch;
  p = Plan{};
  p.scratch = scratch;
}

void Engine::FreePlan() {
  prof_acc_.clear();
  const bool any =
      !plan_.bufs.empty() || in_stage_dev_ || out_stage_dev_ || in_pinned_ || out_pinned_;
  if (any) hipSetDevice(device_);  // frees need the owning device current on this thread
  DrainPrevious();  // the last run may still read or write these buffers
  for (auto& b : plan_.bufs)
    if (b.ptr) hipFree(b.ptr);
  if (in_stage_dev_) hipFree(in_stage_dev_);
  if (out_stage_dev_) hipFree(out_stage_dev_);
  if (in_pinned_) hipHostFree(in_pinned_);
  if (out_pinned_) hipHostFree(out_pinned_);
  in_stage_dev_ = out_stage_dev_ = in_pinned_ = out_pinned_ = nullptr;
  ClearPlan(plan_);
}

void Engine::FreeAll() {
  FreePlan();
  ClearPlan(scratch_plan_);
  if (!wbufs_.empty()) hipSetDevice(device_);
  DrainPrevious();
  for (auto& b : wbufs_)
    if (b.ptr) hipFree(b.ptr);
  wbufs_.clear();
  op_wbuf_.clear();
  op_bbuf_.clear();
  weights_ready_ = false;
}

// Winograd / direct filter transforms for every conv, done once and kept
// across plans (weights do not depend on the input shape).
bool Engine::EnsureWeights(std::string& error) {
  if (weights_ready_) return true;
  auto upload = [&](const void* host, size_t bytes, int& idx) -> bool {
    DevBuf b;
    hipError_t e = hipMalloc(&b.ptr, bytes);
    if (e != hipSuccess) {
      error = "hipMalloc of " + std::to_string(bytes) + " bytes for packed weights failed: " +
              hipGetErrorString(e);
      return false;
    }
    b.bytes = bytes;
    wbufs_.push_back(b);
    idx = static_cast<int>(wbufs_.size()) - 1;
    e = hipMemcpy(b.ptr, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      error = HipErr("hipMemcpy of packed weights", e);
      return false;
    }
    return true;
  };
  for (size_t i = 0; i < graph_.ops.size(); ++i) {
    const Op& op = graph_.ops[i];
    if (op.kind != OpKind::Conv) continue;
    const Weight& w = graph_.weights.at(op.weight);
    const int M = static_cast<int>(w.dims[0]);
    const int C = static_cast<int>(w.dims[1]);
    // Weights are rounded to fp16 first: the model's compute precision.
    std::vector<float> wf(static_cast<size_t>(M) * C * 9);
    for (size_t k = 0; k < wf.size(); ++k) wf[k] = f16_to_f32(f32_to_f16(WeightAt(w, k)));
    std::vector<float> bf(static_cast<size_t>(M), 0.0f);
    if (!op.bias.empty()) {
      const Weight& b = graph_.weights.at(op.bias);
      for (int k = 0; k < M; ++k) bf[k] = f16_to_f32(f32_to_f16(WeightAt(b, k)));
    }
    std::vector<uint16_t> packed;
    if (C == 1) {
      packed.resize(direct_packed_halfs(M));
      direct_pack(wf.data(), M, packed.data());
    } else {
      packed.resize(winograd_packed_halfs(C, M));
      winograd_pack(wf.data(), M, C, packed.data());
    }
    std::vector<float> bias(bias_padded_len(M));
    bias_pad(bf.data(), M, bias.data());
    int wi = -1, bi = -1;
    if (!upload(packed.data(), packed.size() * 2, wi) ||
        !upload(bias.data(), bias.size() * 4, bi)) {
      FreeAll();
      return false;
    }
    op_wbuf_[static_cast<int>(i)] = wi;
    op_bbuf_[static_cast<int>(i)] = bi;
  }
  weights_ready_ = true;
  return true;
}

bool Engine::EnsurePlan(Plan& p, const int64_t in[4], std::string& error, void* scratch,
                        size_t cap) {
  if (p.planned && std::equal(in, in + 4, p.in)) return true;
  if (!built_) {
    error = "engine has no model (build first)";
    return false;
  }
  if (p.scratch)
    ClearPlan(p);  // nothing of a scratch plan is allocated
  else
    FreePlan();
  std::unordered_map<std::string, Shape> shapes;
  if (!PropagateShapes(graph_, in, shapes)) {
    error = "shape propagation failed (unsupported convolution geometry, channel mismatch, "
            "residual/binary operand shape mismatch, or DepthToSpace block size)";
    return false;
  }
  if (!EnsureWeights(error)) return false;

  const auto& ops = graph_.ops;
  const int nops = static_cast<int>(ops.size());
  // Last op index reading each tensor; the graph output lives to the end.
  std::unordered_map<std::string, int> last_use;
  for (int i = 0; i < nops; ++i) {
    last_use[ops[i].in0] = i;
    if (!ops[i].in1.empty()) last_use[ops[i].in1] = i;
    for (const auto& s : ops[i].skips) last_use[s] = i;
  }
  last_use[graph_.output_name] = nops;

  // The final op writes the boundary output itself when it can (a conv, with
  // or without a fused DepthToSpace, or a DepthToSpace) and nothing else
  // reads that tensor; otherwise an output conversion step follows.
  int final_op = -1;
  for (int i = 0; i < nops; ++i)
    if (ops[i].out == graph_.output_name) final_op = i;
  bool output_read_inside = false;
  for (int i = 0; i < nops; ++i) {
    const Op& o = ops[i];
    bool r = o.in0 == graph_.output_name || o.in1 == graph_.output_name;
    for (const auto& s : o.skips) r = r || s == graph_.output_name;
    output_read_inside = output_read_inside || r;
  }
  // A final conv with more than 16 outputs and no fused DepthToSpace or Clip
  // writes the padded layout on the fast body kernels instead; the tiled output
  // conversion then moves it to the boundary (the conv kernels' general
  // boundary epilogue stores one element at a time).
  // The exception is a 64 -> 64 conv without residual inputs that the pipe
  // kernel can store in the fp16 boundary layout itself (pipe_boundary_io).
  bool final_wide = false;
  if (final_op >= 0 && ops[final_op].kind == OpKind::Conv) {
    const Op& fo = ops[final_op];
    const auto& dims = graph_.weights.at(fo.weight).dims;
    final_wide = dims[0] > 16 && fo.dts_b < 1 && !fo.clip;
    const Shape fi = shapes.at(fo.in0);
    if (final_wide && !graph_.output_fp32 && fo.skips.empty() &&
        pipe_boundary_io(fi.n, fi.h, fi.w, dims[1], dims[0], false))
      final_wide = false;
  }
  const bool direct_out = final_op >= 0 && !output_read_inside && !final_wide &&
                          (ops[final_op].kind == OpKind::Conv ||
                           ops[final_op].kind == OpKind::DepthToSpace);

  // Liveness-based buffer reuse (hip_engine.cc:819-898): a buffer is recycled
  // for a tensor of identical padded geometry once every reader of its
  // previous tensor has run. Matching geometry keeps the zero border intact.
  struct Slot {
    int buf;
    int free_after;  // op index of the last reader of the current tensor
    Shape geo;
  };
  std::vector<Slot> slots;
  std::unordered_map<std::string, int> tbuf;  // tensor -> buffer index
  auto alloc = [&](const std::string& name, const Shape& s, int producer) -> bool {
    for (auto& sl : slots) {
      if (sl.free_after < producer && sl.geo == s) {
        sl.free_after = last_use.count(name) ? last_use[name] : producer;
        tbuf[name] = sl.buf;
        return true;
      }
    }
    DevBuf b;
    b.bytes = PaddedBytes(s);
    b.geo = s;
    if (p.scratch) {
      // Laid out in the scratch array at 256-byte alignment; whether the plan
      // fits is checked once the whole layout is known.
      const size_t off = (p.act_bytes + 255) & ~static_cast<size_t>(255);
      b.ptr = off + b.bytes <= cap ? static_cast<char*>(scratch) + off : nullptr;
      p.act_bytes = off + b.bytes;
    } else {
      const hipError_t e = hipMalloc(&b.ptr, b.bytes);
      if (e != hipSuccess) {
        error = "hipMalloc of " + std::to_string(b.bytes) + " bytes for tensor '" + name +
                "' failed: " + hipGetErrorString(e);
        return false;
      }
      p.act_bytes += b.bytes;
    }
    p.bufs.push_back(b);
    p.buf_names.push_back(name);
    const int idx = static_cast<int>(p.bufs.size()) - 1;
    if (!p.scratch) {
      const hipError_t z = hipMemsetAsync(b.ptr, 0, b.bytes, stream_);  // zero border
      if (z != hipSuccess) {
        error = HipErr("hipMemsetAsync of an activation buffer", z);
        return false;
      }
    }
    slots.push_back(Slot{idx, last_use.count(name) ? last_use[name] : producer, s});
    tbuf[name] = idx;
    return true;
  };

  auto fail = [&]() {
    if (p.scratch)
      ClearPlan(p);
    else
      FreePlan();
    return false;
  };

  // Boundary input -> internal padded tensor, unless its only reader is a
  // one-channel head conv on the fast path (padded output, M % 8 == 0, no
  // Clip or residual input), or a 64 -> 64 conv without residual input, Clip
  // or DepthToSpace that the pipe kernel runs on a 64-channel fp16 input
  // (pipe_boundary_io): that conv reads the NCHW boundary input itself.
  const Shape sin = shapes.at(graph_.input_name);
  int fused_in_op = -1;
  if ((sin.c == 1 || sin.c == 64) && graph_.output_name != graph_.input_name) {
    int readers = 0, reader = -1;
    bool other_use = false;
    for (int i = 0; i < nops; ++i) {
      if (ops[i].in0 == graph_.input_name) {
        ++readers;
        reader = i;
      }
      other_use = other_use || ops[i].in1 == graph_.input_name;
      for (const auto& s : ops[i].skips) other_use = other_use || s == graph_.input_name;
    }
    if (readers == 1 && !other_use && ops[reader].kind == OpKind::Conv) {
      const Op& op = ops[reader];
      const int64_t m = graph_.weights.at(op.weight).dims[0];
      const bool to_boundary = direct_out && reader == final_op;
      const bool plain = !op.clip && op.dts_b < 1 && op.skips.empty();
      if (sin.c == 1 && plain && !to_boundary &&
          head_reads_boundary_input(sin.n, sin.h, sin.w, m, graph_.input_fp32))
        fused_in_op = reader;
      // (A 64-channel conv writing the boundary does so through the same pipe.)
      if (sin.c == 64 && plain && !graph_.input_fp32 &&
          pipe_boundary_io(sin.n, sin.h, sin.w, sin.c, m, true))
        fused_in_op = reader;
    }
  }
  if (fused_in_op < 0) {
    if (!alloc(graph_.input_name, sin, -1)) return fail();
    Step st;
    st.kind = StepKind::InputConvert;
    st.in = kBoundaryIn;
    st.out = tbuf[graph_.input_name];
    st.N = (int32_t)sin.n; st.H = (int32_t)sin.h; st.W = (int32_t)sin.w; st.C = (int32_t)sin.c;
    st.fp32 = graph_.input_fp32 ? 1 : 0;
    p.steps.push_back(st);
  }

  const int out_kind_boundary = graph_.output_fp32 ? kOutNchwF32 : kOutNchwF16;
  // Residual-block fusion: conv i (64 -> 64, any activation, no residual
  // input) whose output only conv i + 1 reads, as its input; conv i + 1
  // (64 -> 64, no activation, up to two residual inputs) writes an internal
  // tensor. Both run as one winograd_block launch and conv i's output is never
  // materialized.
  auto readers = [&](const std::string& t) {
    int r = 0;
    for (const Op& o : ops) {
      r += (o.in0 == t) + (o.in1 == t);
      for (const auto& sk : o.skips) r += sk == t;
    }
    return r;
  };
  auto conv_cm = [&](const Op& o, int64_t& c, int64_t& m) {
    const Weight& w = graph_.weights.at(o.weight);
    m = w.dims[0];
    c = w.dims[1];
  };
  auto block_at = [&](int i) -> bool {
    if ((debug_ & kDebugUnfused) || i + 1 >= nops) return false;
    const Op& a = ops[i];
    const Op& b = ops[i + 1];
    if (a.kind != OpKind::Conv || b.kind != OpKind::Conv || i == fused_in_op) return false;
    if (!a.skips.empty() || a.clip || a.dts_b >= 1 || b.clip || b.dts_b >= 1) return false;
    if (b.act != kActNone || b.skips.size() > 2 || b.in0 != a.out) return false;
    if (a.out == graph_.output_name || readers(a.out) != 1) return false;
    if (direct_out && i + 1 == final_op) return false;
    int64_t c1, m1, c2, m2;
    conv_cm(a, c1, m1);
    conv_cm(b, c2, m2);
    if (c1 != 64 || m1 != 64 || c2 != 64 || m2 != 64) return false;
    const Shape si = shapes.at(a.in0);
    return block_eligible(64, 64, a.act, kActNone, si.n, si.h, si.w);
  };
  for (int i = 0; i < nops; ++i) {
    const Op& op = ops[i];
    if (block_at(i)) {
      const Op& op2 = ops[i + 1];
      const Shape si = shapes.at(op.in0);
      // Producer index i: the output must not reuse a buffer conv i reads.
      if (!alloc(op2.out, shapes.at(op2.out), i)) return fail();
      Step st;
      st.kind = StepKind::ConvBlock;
      st.op = i;
      st.op2 = i + 1;
      st.in = tbuf.at(op.in0);
      st.out = tbuf.at(op2.out);
      st.N = (int32_t)si.n; st.H = (int32_t)si.h; st.W = (int32_t)si.w; st.C = 64; st.M = 64;
      st.wbuf = op_wbuf_.at(i);
      st.bbuf = op_bbuf_.at(i);
      st.wbuf2 = op_wbuf_.at(i + 1);
      st.bbuf2 = op_bbuf_.at(i + 1);
      for (size_t k = 0; k < op2.skips.size(); ++k) st.skip[k] = tbuf.at(op2.skips[k]);
      st.epi.act = op.act;
      p.steps.push_back(st);
      ++i;
      continue;
    }
    const Shape si = shapes.at(op.in0);
    const Shape so = shapes.at(op.out);
    const bool to_boundary = direct_out && i == final_op;
    int out_buf = kBoundaryOut;
    if (!to_boundary && !alloc(op.out, so, i)) return fail();
    if (!to_boundary) out_buf = tbuf[op.out];

    Step st;
    st.op = i;
    if (i == fused_in_op) {
      st.in = kBoundaryIn;
      st.in_kind = graph_.input_fp32 ? 2 : 1;
    } else {
      st.in = tbuf.at(op.in0);
    }
    st.out = out_buf;
    st.N = (int32_t)si.n; st.H = (int32_t)si.h; st.W = (int32_t)si.w; st.C = (int32_t)si.c;
    switch (op.kind) {
      case OpKind::Conv: {
        const Weight& w = graph_.weights.at(op.weight);
        st.M = static_cast<int32_t>(w.dims[0]);
        st.kind = st.C == 1 ? StepKind::ConvDirect : StepKind::ConvWinograd;
        st.wbuf = op_wbuf_.at(i);
        st.bbuf = op_bbuf_.at(i);
        for (size_t k = 0; k < op.skips.size(); ++k) st.skip[k] = tbuf.at(op.skips[k]);
        st.epi.act = op.act;
        st.epi.out_kind = to_boundary ? out_kind_boundary : kOutPadded;
        st.epi.dts_b = (to_boundary && op.dts_b >= 2) ? op.dts_b : 0;
        st.epi.do_clip = op.clip ? 1 : 0;
        st.epi.clip_lo = op.clip_lo;
        st.epi.clip_hi = op.clip_hi;
        if (op.dts_b >= 1 && !to_boundary) {
          error = "internal error: fused DepthToSpace conv does not write the graph output";
          return fail();
        }
        break;
      }
      case OpKind::Sigmoid:
      case OpKind::Relu:
      case OpKind::Clip:
        st.kind = StepKind::Eltwise;
        st.elt_op = op.kind == OpKind::Sigmoid ? kUnarySigmoid
                    : op.kind == OpKind::Relu  ? kUnaryRelu
                                               : kUnaryClip;
        st.lo = op.clip_lo;
        st.hi = op.clip_hi;
        if (to_boundary) {
          error = "internal error: elementwise op cannot write the boundary";
          return fail();
        }
        break;
      case OpKind::Add:
      case OpKind::Mul:
        st.kind = StepKind::Eltwise;
        st.binary = true;
        st.elt_op = op.kind == OpKind::Mul ? kBinaryMul : kBinaryAdd;
        st.in2 = tbuf.at(op.in1);
        break;
      case OpKind::DepthToSpace:
        st.kind = StepKind::DepthToSpace;
        st.dts_b = op.blocksize;
        st.out_kind = to_boundary ? out_kind_boundary : kOutPadded;
        st.do_clip = op.clip ? 1 : 0;
        st.lo = op.clip_lo;
        st.hi = op.clip_hi;
        break;
    }
    p.steps.push_back(st);
  }

  if (!direct_out) {
    const Shape so = shapes.at(graph_.output_name);
    Step st;
    st.kind = StepKind::OutputConvert;
    st.in = tbuf.at(graph_.output_name);
    st.out = kBoundaryOut;
    st.N = (int32_t)so.n; st.H = (int32_t)so.h; st.W = (int32_t)so.w; st.C = (int32_t)so.c;
    st.fp32 = graph_.output_fp32 ? 1 : 0;
    p.steps.push_back(st);
  }

  // A block stores its output with plain stores (not non-temporal) when the
  // next step is bound by HBM and the output fits the 256 MiB last-level
  // cache (Infinity Cache) about once, so that this reader finds much of it
  // still cached. HBM-bound readers: a conv writing the boundary output (the
  // tail), a conv with residual inputs, and the elementwise and layout passes.
  // Another block, or a conv without residual inputs into padded NHWC, is
  // bound by its own arithmetic and gains nothing, while plain stores cost the
  // writing block ~1-4 us. At 1080p (266 MB): R8F64's tail 64 -> 55 us, the
  // shipped architecture's residual conv after its last block 167 -> 157 us,
  // both frames ~0.2% faster. At 4K x 2 (2.1 GB) the tail slowed 483 -> 493 us.
  constexpr int64_t kCachedOutMax = 320ll << 20;
  auto hbm_bound = [](const Step& n) {
    switch (n.kind) {
      case StepKind::ConvBlock: return false;
      case StepKind::ConvWinograd:
      case StepKind::ConvDirect:
        return n.epi.out_kind != kOutPadded || n.skip[0] != kNoBuffer;
      default: return true;
    }
  };
  for (size_t j = 0; j + 1 < p.steps.size(); ++j) {
    Step& st = p.steps[j];
    if (st.kind != StepKind::ConvBlock) continue;
    const int64_t out_bytes = (int64_t)st.N * padded_rows(st.H) * padded_cols(st.W) * st.M * 2;
    st.cached_out = out_bytes <= kCachedOutMax && hbm_bound(p.steps[j + 1]);
  }

  p.in_bytes = static_cast<size_t>(in[0] * in[1] * in[2] * in[3]) * (graph_.input_fp32 ? 4 : 2);
  p.out_bytes = OutputBytesUnlocked(in);
  if (p.scratch) {
    if (p.act_bytes > cap) {
      error = "the activations of a " + std::to_string(in[0]) + "x" + std::to_string(in[1]) +
              "x" + std::to_string(in[2]) + "x" + std::to_string(in[3]) + " input need " +
              std::to_string(p.act_bytes) + " bytes; the no-allocation scratch holds " +
              std::to_string(cap) + " bytes (use arthip_engine_run_device for larger inputs)";
      return fail();
    }
  } else {
    const hipError_t e = hipStreamSynchronize(stream_);  // buffer zeroing done
    if (e != hipSuccess) {
      error = HipErr("hipStreamSynchronize after plan setup", e);
      return fail();
    }
  }
  std::copy(in, in + 4, p.in);
  p.planned = true;
  // VSHIP_DEBUG (hip_engine.cc:1167-1184): the new plan's launches.
  if (debug_ & kDebugPlan) {
    Log("[vship] %s for [%lld,%lld,%lld,%lld]: %zu launches, %zu activation buffers, %zu "
        "bytes\n", p.scratch ? "scratch plan" : "plan", (long long)in[0], (long long)in[1],
        (long long)in[2], (long long)in[3], p.steps.size(), p.bufs.size(), p.act_bytes);
    for (size_t i = 0; i < p.steps.size(); ++i) {
      const Step& st = p.steps[i];
      Log("[vship] step%-2zu %s in=%d in2=%d skip=%d,%d out=%d\n", i, StepName(st).c_str(),
          st.in, st.in2, st.skip[0], st.skip[1], st.out);
    }
  }
  return true;
}

bool Engine::Enqueue(const Plan& p, const void* in_dev, void* out_dev, hipStream_t s,
                     std::string& error) {
  auto ptr = [&](int idx) -> void* {
    if (idx == kBoundaryIn) return const_cast<void*>(in_dev);
    if (idx == kBoundaryOut) return out_dev;
    if (idx < 0) return nullptr;
    return p.bufs[idx].ptr;
  };
  auto bytes_of = [&](int idx) -> size_t {
    if (idx == kBoundaryIn) return p.in_bytes;
    if (idx == kBoundaryOut) return p.out_bytes;
    if (idx < 0) return 0;
    return p.bufs[idx].bytes;
  };
  // A run on a capturing stream becomes graph nodes that execute at each
  // replay. It cannot wait on the previous run's event (recorded outside the
  // capture), so that run must be over; it records no end event (the caller
  // orders the replays); and it neither synchronizes (VSHIP_SYNC_EACH is
  // refused), nor times its launches, nor dumps.
  bool capturing = false;
  if (!StreamCapturing(s, capturing, error)) return false;
  RelaxedCaptureMode relax(capturing);
  if (capturing && (debug_ & kDebugSyncEach)) {
    error = "VSHIP_SYNC_EACH synchronizes the stream after every launch, which a stream under "
            "HIP graph capture does not allow";
    return false;
  }
  // Profiling events and dumps create events and host buffers: runs on a
  // scratch plan do neither.
  const bool profiling = profiling_ && !p.scratch && !capturing;
  if (profiling && prof_acc_.size() != p.steps.size()) {
    prof_acc_.assign(p.steps.size(), StepProfile{});
    for (size_t i = 0; i < p.steps.size(); ++i) prof_acc_[i].name = StepName(p.steps[i]);
  }
  if (capturing ? !PreviousDone(error) : !WaitPrevious(s, error)) return false;
  // From here on the run's work is on s: later runs order after it even when
  // this one fails part way.
  if (!capturing) last_stream_ = s;
  auto finish = [&](bool ok) -> bool {
    if (capturing) return ok;
    const hipError_t r = hipEventRecord(run_done_, s);
    if (r != hipSuccess && ok) {
      error = HipErr("hipEventRecord at the end of a run", r);
      return false;
    }
    return ok;
  };

  // A scratch plan's buffers hold whatever the last user of the scratch array
  // left: clear their borders, the zero padding every conv reads, with a
  // kernel (no memset node for callers that capture the stream).
  if (p.scratch) {
    for (const DevBuf& b : p.bufs) {
      const hipError_t e = launch_zero_border(b.ptr, (int32_t)b.geo.n, (int32_t)b.geo.h,
                                              (int32_t)b.geo.w, (int32_t)b.geo.c, s);
      if (e != hipSuccess) {
        error = HipErr("scratch border clear", e);
        return finish(false);
      }
    }
  }
  // VSHIP_POISON: every activation interior becomes fp16 NaN (0x7E7E), the
  // reference's poison pattern; the zero border stays. A launch that reads a
  // tensor no earlier launch of this run wrote then yields NaN.
  if (debug_ & kDebugPoison) {
    for (const DevBuf& b : p.bufs) {
      const hipError_t e = launch_poison(b.ptr, (int32_t)b.geo.n, (int32_t)b.geo.h,
                                         (int32_t)b.geo.w, (int32_t)b.geo.c, 0x7E7E, s);
      if (e != hipSuccess) {
        error = HipErr("poison fill", e);
        return finish(false);
      }
    }
  }
  // VSHIP_DUMP: each launch's inputs and output as raw files, for the first
  // two runs of the engine. Activations are padded NHWC fp16 buffers.
  const bool dump = !p.scratch && !capturing && (debug_ & kDebugDump) != 0 &&
                    !dump_dir_.empty() && dump_runs_ < 2;
  const uint64_t dump_run = dump ? ++dump_runs_ : 0;

  for (size_t i = 0; i < p.steps.size(); ++i) {
    const Step& st = p.steps[i];
    hipError_t e = hipSuccess;
    EventPair ev{static_cast<int>(i), nullptr, nullptr};
    if (profiling) {
      ev.start = TakeEvent();
      ev.stop = TakeEvent();
      if (ev.start == nullptr || ev.stop == nullptr || hipEventRecord(ev.start, s) != hipSuccess) {
        error = "HIP event creation/record for profiling failed";
        return finish(false);
      }
    }
    switch (st.kind) {
      case StepKind::InputConvert:
      case StepKind::OutputConvert: {
        IoArgs a{};
        a.src = ptr(st.in);
        a.dst = ptr(st.out);
        a.N = st.N; a.H = st.H; a.W = st.W; a.C = st.C;
        a.Hp = (int32_t)padded_rows(st.H);
        a.Wp = (int32_t)padded_cols(st.W);
        a.fp32 = st.fp32;
        e = st.kind == StepKind::InputConvert ? launch_input_convert(a, s)
                                              : launch_output_convert(a, s);
        break;
      }
      case StepKind::ConvWinograd:
      case StepKind::ConvDirect: {
        Epilogue epi = st.epi;
        epi.bias = static_cast<const float*>(wbufs_[st.bbuf].ptr);
        epi.skip0 = static_cast<const uint16_t*>(ptr(st.skip[0]));
        epi.skip1 = static_cast<const uint16_t*>(ptr(st.skip[1]));
        epi.out = ptr(st.out);
        if (st.kind == StepKind::ConvDirect) {
          DirectArgs a{};
          a.in = ptr(st.in);
          a.in_kind = st.in_kind;
          a.w = static_cast<const uint16_t*>(wbufs_[st.wbuf].ptr);
          a.epi = epi;
          a.N = st.N; a.H = st.H; a.W = st.W; a.M = st.M;
          e = launch_direct(a, s);
        } else {
          WinoArgs a{};
          a.in = static_cast<const uint16_t*>(ptr(st.in));
          a.in_nchw = st.in == kBoundaryIn ? 1 : 0;
          a.u = static_cast<const uint16_t*>(wbufs_[st.wbuf].ptr);
          a.epi = epi;
          a.N = st.N; a.H = st.H; a.W = st.W; a.C = st.C; a.M = st.M;
          e = launch_winograd(a, s);
        }
        break;
      }
      case StepKind::ConvBlock: {
        BlockArgs a{};
        a.in = static_cast<const uint16_t*>(ptr(st.in));
        a.u1 = static_cast<const uint16_t*>(wbufs_[st.wbuf].ptr);
        a.bias1 = static_cast<const float*>(wbufs_[st.bbuf].ptr);
        a.u2 = static_cast<const uint16_t*>(wbufs_[st.wbuf2].ptr);
        a.bias2 = static_cast<const float*>(wbufs_[st.bbuf2].ptr);
        a.skip0 = static_cast<const uint16_t*>(ptr(st.skip[0]));
        a.skip1 = static_cast<const uint16_t*>(ptr(st.skip[1]));
        a.out = static_cast<uint16_t*>(ptr(st.out));
        a.N = st.N; a.H = st.H; a.W = st.W;
        a.act1 = st.epi.act;
        a.act2 = kActNone;
        a.cached_out = st.cached_out ? 1 : 0;
        e = launch_block(a, s);
        break;
      }
      case StepKind::Eltwise: {
        EltArgs a{};
        a.a = static_cast<const uint16_t*>(ptr(st.in));
        a.b = static_cast<const uint16_t*>(ptr(st.in2));
        a.out = static_cast<uint16_t*>(ptr(st.out));
        a.N = st.N; a.H = st.H; a.W = st.W; a.C = st.C;
        a.Hp = (int32_t)padded_rows(st.H);
        a.Wp = (int32_t)padded_cols(st.W);
        a.op = st.elt_op;
        a.lo = st.lo;
        a.hi = st.hi;
        e = launch_eltwise(a, st.binary, s);
        break;
      }
      case StepKind::DepthToSpace: {
        DtsArgs a{};
        a.in = static_cast<const uint16_t*>(ptr(st.in));
        a.out = ptr(st.out);
        a.N = st.N; a.H = st.H; a.W = st.W; a.C = st.C;
        a.Hp = (int32_t)padded_rows(st.H);
        a.Wp = (int32_t)padded_cols(st.W);
        a.b = st.dts_b;
        a.out_kind = st.out_kind;
        a.do_clip = st.do_clip;
        a.lo = st.lo;
        a.hi = st.hi;
        e = launch_dts(a, s);
        break;
      }
    }
    if (e != hipSuccess) {
      error = "HIP kernel launch for step " + std::to_string(i) + " failed: " +
              hipGetErrorString(e);
      return finish(false);
    }
    if (debug_ & kDebugTrace)
      Log("[run] #%llu op%zu %s\n", (unsigned long long)run_no_, i, StepName(st).c_str());
    if (debug_ & kDebugDumpOps) {
      std::string line = "[dump] op " + std::to_string(i) + " " + StepName(st) + " in=";
      for (int idx : {st.in, st.in2, st.skip[0], st.skip[1]})
        if (idx != kNoBuffer) line += BufLabel(p, idx, in_dev, out_dev) + " ";
      line += "out=" + BufLabel(p, st.out, in_dev, out_dev);
      Log("%s\n", line.c_str());
    }
    if (profiling) {
      if (hipEventRecord(ev.stop, s) != hipSuccess) {
        error = "HIP event record for profiling failed";
        return finish(false);
      }
      pending_events_.push_back(ev);
    }
    if (debug_ & kDebugSyncEach) {
      const hipError_t se = hipStreamSynchronize(s);
      if (se != hipSuccess) {
        error = HipErr(("sync-each after step " + std::to_string(i)).c_str(), se);
        return finish(false);
      }
    }
    if (dump) {
      const int ins[4] = {st.in, st.in2, st.skip[0], st.skip[1]};
      int k = 0;
      char path[4096];
      for (int idx : ins) {
        if (idx == kNoBuffer) continue;
        std::snprintf(path, sizeof(path), "%s/run%llu_op%02zu_in%d.bin", dump_dir_.c_str(),
                      (unsigned long long)dump_run, i, k++);
        if (!Dump(path, ptr(idx), bytes_of(idx), s)) {
          error = std::string("dump of ") + path + " failed";
          return finish(false);
        }
      }
      std::snprintf(path, sizeof(path), "%s/run%llu_op%02zu_out.bin", dump_dir_.c_str(),
                    (unsigned long long)dump_run, i);
      if (!Dump(path, ptr(st.out), bytes_of(st.out), s)) {
        error = std::string("dump of ") + path + " failed";
        return finish(false);
      }
    }
  }
  return finish(true);
}

bool Engine::Dump(const std::string& path, const void* dev, size_t bytes, hipStream_t s) {
  std::vector<uint8_t> host(bytes);
  hipError_t e = hipMemcpyAsync(host.data(), dev, bytes, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return false;
  FILE* f = std::fopen(path.c_str(), "wb");
  if (f == nullptr) return false;
  const bool ok = std::fwrite(host.data(), 1, bytes, f) == bytes;
  return std::fclose(f) == 0 && ok;
}

hipEvent_t Engine::TakeEvent() {
  if (!event_pool_.empty()) {
    hipEvent_t e = event_pool_.back();
    event_pool_.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

std::string Engine::StepName(const Step& st) const {
  static const char* acts[] = {"", " relu", " silu"};
  std::ostringstream os;
  switch (st.kind) {
    case StepKind::InputConvert: os << "input_convert C" << st.C; break;
    case StepKind::OutputConvert: os << "output_convert C" << st.C; break;
    case StepKind::ConvWinograd:
    case StepKind::ConvDirect:
      os << (st.kind == StepKind::ConvWinograd ? "winograd_conv" : "direct_conv") << " C" << st.C
         << " M" << st.M << acts[st.epi.act];
      for (int k = 0; k < 2; ++k)
        if (st.skip[k] != kNoBuffer) os << " +skip";
      if (st.epi.dts_b) os << " +dts" << st.epi.dts_b;
      if (st.epi.do_clip) os << " +clip";
      break;
    case StepKind::ConvBlock:
      os << "winograd_block C64 M64" << acts[st.epi.act];
      for (int k = 0; k < 2; ++k)
        if (st.skip[k] != kNoBuffer) os << " +skip";
      if (st.cached_out) os << " +cached_out";
      break;
    case StepKind::Eltwise: os << "eltwise op" << st.elt_op << (st.binary ? " binary" : ""); break;
    case StepKind::DepthToSpace: os << "depth_to_space b" << st.dts_b; break;
  }
  os << " [" << st.N << "x" << st.H << "x" << st.W << "]";
  return os.str();
}

void Engine::SetProfiling(bool on) {
  std::lock_guard<std::mutex> lock(mu_);
  profiling_ = on;
  prof_acc_.clear();
}

bool Engine::ProfileRead(std::vector<StepProfile>& out, std::string& error) {
  std::lock_guard<std::mutex> lock(mu_);
  for (const EventPair& ev : pending_events_) {
    hipError_t e = hipEventSynchronize(ev.stop);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.start, ev.stop);
    if (e != hipSuccess) {
      error = HipErr("hipEventElapsedTime", e);
      return false;
    }
    if (ev.step < static_cast<int>(prof_acc_.size())) {
      prof_acc_[ev.step].total_ms += ms;
      prof_acc_[ev.step].launches += 1;
    }
    event_pool_.push_back(ev.start);
    event_pool_.push_back(ev.stop);
  }
  pending_events_.clear();
  out = prof_acc_;
  for (auto& p : prof_acc_) {
    p.total_ms = 0.0;
    p.launches = 0;
  }
  return true;
}

bool Engine::Run(const void* in_host, const int64_t in[4], void* out_host, size_t out_cap,
                 std::string& error) {
  std::lock_guard<std::mutex> lock(mu_);
  RunLog rl(*this, "run", in_host, true, error);
  (void)hipGetLastError();  // a stale error from an earlier failed call is not this run's
  if (!Init(error)) return false;
  if (!EnsurePlan(plan_, in, error)) return false;
  rl.Built();
  const size_t in_bytes = plan_.in_bytes, out_bytes = plan_.out_bytes;
  if (in_host == nullptr || out_host == nullptr) {
    error = "null host buffer";
    return false;
  }
  if (out_cap < out_bytes) {
    error = "output buffer too small (" + std::to_string(out_cap) + " bytes, need " +
            std::to_string(out_bytes) + ")";
    return false;
  }
  hipError_t e;
  if (in_stage_dev_ == nullptr) {
    if ((e = hipMalloc(&in_stage_dev_, in_bytes)) != hipSuccess ||
        (e = hipMalloc(&out_stage_dev_, out_bytes)) != hipSuccess ||
        (e = hipHostMalloc(&in_pinned_, in_bytes, hipHostMallocDefault)) != hipSuccess ||
        (e = hipHostMalloc(&out_pinned_, out_bytes, hipHostMallocDefault)) != hipSuccess) {
      error = "hipMalloc of IO staging failed: " + std::string(hipGetErrorString(e));
      FreePlan();
      return false;
    }
  }
  std::memcpy(in_pinned_, in_host, in_bytes);
  if ((e = hipMemcpyAsync(in_stage_dev_, in_pinned_, in_bytes, hipMemcpyHostToDevice,
                          stream_)) != hipSuccess) {
    error = HipErr("HIP input upload", e);
    return false;
  }
  rl.Uploaded();
  if (!Enqueue(plan_, in_stage_dev_, out_stage_dev_, stream_, error)) return false;
  rl.Launched();
  if ((e = hipMemcpyAsync(out_pinned_, out_stage_dev_, out_bytes, hipMemcpyDeviceToHost,
                          stream_)) != hipSuccess) {
    error = HipErr("HIP output download", e);
    return false;
  }
  if ((e = hipStreamSynchronize(stream_)) != hipSuccess) {
    error = HipErr("HIP stream synchronize", e);
    return false;
  }
  rl.Back();
  std::memcpy(out_host, out_pinned_, out_bytes);
  return rl.Done(out_host);
}

bool Engine::RunDevice(const void* in_dev, const int64_t in[4], void* out_dev,
                       hipStream_t stream, std::string& error) {
  std::lock_guard<std::mutex> lock(mu_);
  RunLog rl(*this, "run_device", in_dev, false, error);
  (void)hipGetLastError();
  if (!Init(error)) return false;
  if (!EnsurePlan(plan_, in, error)) return false;
  rl.Built();
  if (in_dev == nullptr || out_dev == nullptr) {
    error = "null device buffer";
    return false;
  }
  if (!Enqueue(plan_, in_dev, out_dev, stream ? stream : stream_, error)) return false;
  rl.Launched();
  return rl.Done(out_dev);
}

bool Engine::RunDeviceScratch(const void* in_dev, const int64_t in[4], void* out_dev,
                              hipStream_t stream, std::string& error) {
  std::lock_guard<std::mutex> lock(mu_);
  RunLog rl(*this, "run_device_noalloc", in_dev, false, error);
  (void)hipGetLastError();
  if (stream_ == nullptr || run_done_ == nullptr || !weights_ready_) {
    error = "the engine is not set up on its device yet: one run (arthip_engine_run or "
            "arthip_engine_run_device, any input size) creates its stream and uploads its "
            "weights; the no-allocation entry point does neither";
    return false;
  }
  if (!SetDevice(error)) return false;
  if (in_dev == nullptr || out_dev == nullptr) {
    error = "null device buffer";
    return false;
  }
  const hipStream_t s = stream ? stream : stream_;
  bool capturing = false;
  if (!StreamCapturing(s, capturing, error)) return false;
  RelaxedCaptureMode relax(capturing);
  // Every handle on this device shares its scratch: the lease orders this
  // call after the last one that used it (and holds off the next) until End.
  ScratchUse use;
  void* scratch = nullptr;
  if (!use.Begin(device_, s, capturing, &scratch, error)) return false;
  scratch_plan_.scratch = true;
  if (!EnsurePlan(scratch_plan_, in, error, scratch, kNoAllocScratchBytes)) return false;
  rl.Built();
  const bool ok = Enqueue(scratch_plan_, in_dev, out_dev, s, error);
  std::string end_error;
  if (!use.End(end_error) && ok) {
    error = end_error;
    return false;
  }
  if (!ok) return false;
  rl.Launched();
  return rl.Done(out_dev);
}

std::string Engine::Describe() const {
  std::lock_guard<std::mutex> lock(mu_);
  std::ostringstream os;
  os << "input '" << graph_.input_name << "'" << (graph_.input_fp32 ? " fp32" : " fp16")
     << ", output '" << graph_.output_name << "'" << (graph_.output_fp32 ? " fp32" : " fp16")
     << "\n";
  static const char* acts[] = {"", "+relu", "+silu"};
  for (size_t i = 0; i < graph_.ops.size(); ++i) {
    const Op& op = graph_.ops[i];
    os << "op" << i << " " << OpKindName(op.kind);
    if (op.kind == OpKind::Conv) {
      const Weight& w = graph_.weights.at(op.weight);
      os << " " << w.dims[1] << "->" << w.dims[0] << acts[op.act];
      for (const auto& s : op.skips) os << " +skip(" << s << ")";
      if (op.dts_b) os << " +dts" << op.dts_b;
    }
    if (op.clip) os << " +clip[" << op.clip_lo << "," << op.clip_hi << "]";
    os << " : " << op.in0 << (op.in1.empty() ? "" : ", " + op.in1) << " -> " << op.out << "\n";
  }
  for (const Plan* p : {&plan_, &scratch_plan_}) {
    if (!p->planned) continue;
    os << (p->scratch ? "scratch plan" : "plan") << " for [" << p->in[0] << "," << p->in[1]
       << "," << p->in[2] << "," << p->in[3] << "]: " << p->steps.size() << " launches, "
       << p->bufs.size() << " activation buffers: " << p->act_bytes << " bytes\n";
  }
  return os.str();
}

}  // namespace arthip
