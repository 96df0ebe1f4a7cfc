// The conv-chain engine: one compiled model on one GPU.
//
// Replaces vship::HipEngine (src/vapoursynth/hip_engine.h:88-188) and
// onnxruntime::hip::HipGraph (src/onnxruntime-hip/hip_graph.h:113-167) with a
// single core both adapters can drive: Build parses and fuses an ONNX model;
// a per-input-shape plan (buffers, packed weights, launch list) is built on
// first use and cached; Run executes one batch host-to-host, RunDevice on
// device-resident buffers. Thread-safe through an internal mutex; every entry
// point re-selects the device (HIP's current device is per thread).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "conv_args.h"
#include "graph.h"

namespace arthip {

struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  Shape geo{};  // activation buffers: the tensor geometry (padded NHWC around it)
};

// Diagnostics, the reference's environment switches (hip_engine.cc:1167-1184,
// 1280-1289,1310-1349; hip_graph.cc:131-132,1213-1447,1231-1248,1356-1373). An
// engine starts from VSHIP_POISON=1, VSHIP_SYNC_EACH=1, VSHIP_DUMP=<dir>,
// VSHIP_TRACE=1, HIP_PROFILE=1, HIP_DUMPOPS (set) and VSHIP_DEBUG=1; SetDebug
// overrides them. The last four write lines to the engine's log (stderr
// unless SetLog names a file).
enum DebugFlag : int {
  kDebugPoison = 1,       // before each run, fill every activation interior with fp16 NaN
  kDebugSyncEach = 2,     // synchronize the launch stream after every launch
  kDebugDump = 4,         // write each launch's inputs and output (first two runs)
  kDebugUnfused = 8,      // run every conv as its own launch (no residual-block fusion)
  kDebugTrace = 16,       // "[run]" lines: enter, plan ready, each launch, done / fail
  kDebugHostProfile = 32, // "[hipprof]" host time spans of each run
  kDebugDumpOps = 64,     // "[dump]" line per launch: its buffers, addresses and sizes
  kDebugPlan = 128,       // "[vship]" lines describing each new plan's launches
};
constexpr int kDebugAll = kDebugPoison | kDebugSyncEach | kDebugDump | kDebugUnfused |
                          kDebugTrace | kDebugHostProfile | kDebugDumpOps | kDebugPlan;

enum class StepKind {
  InputConvert,
  ConvWinograd,
  ConvDirect,
  ConvBlock,  // two 64 -> 64 convs fused (winograd_block): op, op2
  Eltwise,
  DepthToSpace,
  OutputConvert
};

// Buffer reference inside a plan: an index into Engine::bufs_, or the
// boundary input/output supplied per run.
constexpr int kBoundaryIn = -2;
constexpr int kBoundaryOut = -3;
constexpr int kNoBuffer = -1;

struct Step {
  StepKind kind = StepKind::ConvWinograd;
  int op = -1;   // index into Graph::ops (-1 for IO steps)
  int op2 = -1;  // ConvBlock: the second conv
  int in = kNoBuffer, in2 = kNoBuffer, out = kNoBuffer;
  int skip[2] = {kNoBuffer, kNoBuffer};
  int wbuf = kNoBuffer, bbuf = kNoBuffer;  // packed weights / padded bias (weight cache)
  int wbuf2 = kNoBuffer, bbuf2 = kNoBuffer;  // ConvBlock: the second conv's
  // Geometry of the step's input (NHWC) and channel counts.
  int32_t N = 0, H = 0, W = 0, C = 0, M = 0;
  Epilogue epi{};  // conv epilogue (pointers resolved per run)
  int32_t elt_op = 0;
  bool binary = false;
  int32_t dts_b = 0, out_kind = kOutPadded, do_clip = 0;
  float lo = 0.0f, hi = 0.0f;
  int32_t fp32 = 0;  // IO steps: boundary side is fp32
  int32_t in_kind = 0;  // direct conv reading the boundary input: 1 fp16, 2 fp32
  bool cached_out = false;  // ConvBlock: plain output stores (the next step is HBM-bound)
};

// One input shape's launch list and activation buffers.
struct Plan {
  bool planned = false;
  bool scratch = false;  // activations live in the no-allocation scratch array
  int64_t in[4] = {0, 0, 0, 0};
  std::vector<DevBuf> bufs;
  std::vector<Step> steps;
  std::vector<std::string> buf_names;
  size_t in_bytes = 0, out_bytes = 0;
  size_t act_bytes = 0;  // activation bytes (for a scratch plan: the extent used)
};

class Engine {
 public:
  explicit Engine(int device_id);
  ~Engine();
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  // Selects the device and creates the engine's stream (once; later calls
  // only re-select the device). Run / RunDevice call it; Build does not, so
  // models can be parsed and validated without a GPU.
  bool Init(std::string& error);

  bool Build(const void* data, size_t size, std::string& error,
             const BuildOptions& opts = BuildOptions());
  bool BuildFile(const std::string& path, std::string& error,
                 const BuildOptions& opts = BuildOptions());
  bool BuildParsed(const onnx::Model& model, std::string& error,
                   const BuildOptions& opts = BuildOptions());

  bool OutputShape(const int64_t in_nchw[4], int64_t out_nchw[4]) const;
  bool InputFp32() const;
  bool OutputFp32() const;
  // First conv's input channels / last conv's output channels (before a
  // trailing DepthToSpace), as the reference reports them (hip_engine.h:127-136).
  int InputChannels() const;
  int OutputChannels() const;

  bool Run(const void* in_host, const int64_t in_nchw[4], void* out_host, size_t out_cap,
           std::string& error);
  // RunDevice enqueues on `stream` (null: the engine's stream) and returns
  // without waiting. Runs on one engine share its activation buffers, so each
  // run's launches are ordered after the previous run's, whatever streams the
  // two were given (an event recorded at the end of every run, waited on by
  // the next run's stream when it differs).
  bool RunDevice(const void* in_dev, const int64_t in_nchw[4], void* out_dev, hipStream_t stream,
                 std::string& error);

  // RunDevice without any device allocation: the activations go to `scratch`
  // (scratch_cap bytes of device memory that the caller owns for the call) in
  // a plan of their own; borders are cleared by a kernel each run. Needs the
  // engine initialized and its weights resident (any earlier Run / RunDevice
  // does both). Not profiled and not dumped.
  bool RunDeviceScratch(const void* in_dev, const int64_t in_nchw[4], void* out_dev,
                        hipStream_t stream, std::string& error);
  int Device() const { return device_; }

  // Diagnostics (DebugFlag bits); dump_dir is used with kDebugDump.
  void SetDebug(int flags, const std::string& dump_dir);
  int DebugFlags() const;
  // Where the trace, host-profile, op-dump and plan lines go: appended to the
  // file at `path`, or stderr for an empty path.
  bool SetLog(const std::string& path, std::string& error);

  std::string Describe() const;

  // Per-launch GPU timing with HIP events recorded around every step on the
  // launch stream (the reference's VSHIP_PROFILE, hip_engine.cc:1409-1606).
  // ProfileRead synchronizes the recorded events and returns, per plan step,
  // the summed milliseconds and launch count since the last read.
  void SetProfiling(bool on);
  struct StepProfile {
    std::string name;
    double total_ms = 0.0;
    int64_t launches = 0;
  };
  bool ProfileRead(std::vector<StepProfile>& out, std::string& error);
  size_t InputBytes(const int64_t in_nchw[4]) const;
  size_t OutputBytes(const int64_t in_nchw[4]) const;

 private:
  bool SetDevice(std::string& error) const;
  bool OutputShapeUnlocked(const int64_t in_nchw[4], int64_t out_nchw[4]) const;
  size_t OutputBytesUnlocked(const int64_t in_nchw[4]) const;
  // Builds p for this input shape (cached per shape). With p.scratch the
  // activations are laid out from `scratch` (cap bytes) and nothing is
  // allocated; otherwise each buffer is a zeroed hipMalloc.
  bool EnsurePlan(Plan& p, const int64_t in_nchw[4], std::string& error, void* scratch = nullptr,
                  size_t cap = 0);
  bool EnsureWeights(std::string& error);
  bool Enqueue(const Plan& p, const void* in_dev, void* out_dev, hipStream_t s,
               std::string& error);
  static void ClearPlan(Plan& p);
  void FreePlan();  // the allocated plan and the host-path staging
  void FreeAll();

  int device_;
  hipStream_t stream_ = nullptr;
  // Completion of the last enqueued run and the stream it went to.
  hipEvent_t run_done_ = nullptr;
  hipStream_t last_stream_ = nullptr;
  bool WaitPrevious(hipStream_t s, std::string& error);
  bool PreviousDone(std::string& error);
  bool DrainPrevious();

  int debug_ = 0;
  std::string dump_dir_;
  uint64_t dump_runs_ = 0;
  FILE* log_ = nullptr;  // null: stderr
  uint64_t run_no_ = 0;  // runs seen by the trace (kDebugTrace)
  void Log(const char* fmt, ...) __attribute__((format(printf, 2, 3)));
  std::string BufLabel(const Plan& p, int idx, const void* in_dev, const void* out_dev) const;
  // kDebugTrace / kDebugHostProfile bookkeeping of one Run / RunDevice call.
  struct RunLog;
  bool Dump(const std::string& path, const void* dev, size_t bytes, hipStream_t s);
  Graph graph_;
  bool built_ = false;

  // Packed weights, shape independent; uploaded on the first plan.
  bool weights_ready_ = false;
  std::vector<DevBuf> wbufs_;
  std::unordered_map<int, int> op_wbuf_, op_bbuf_;  // op index -> wbufs_ index

  // Current plans: allocated activations (Run, RunDevice) and activations in
  // the scratch array (RunDeviceScratch).
  Plan plan_;
  Plan scratch_plan_;
  // Host Run path: device copies of the boundary tensors and pinned staging.
  void* in_stage_dev_ = nullptr;
  void* out_stage_dev_ = nullptr;
  void* in_pinned_ = nullptr;
  void* out_pinned_ = nullptr;

  // Profiling: event pairs (step index, start, stop) not yet read.
  bool profiling_ = false;
  struct EventPair {
    int step;
    hipEvent_t start, stop;
  };
  std::vector<EventPair> pending_events_;
  std::vector<hipEvent_t> event_pool_;
  std::vector<StepProfile> prof_acc_;
  hipEvent_t TakeEvent();
  std::string StepName(const Step& st) const;

  mutable std::mutex mu_;
};

}  // namespace arthip
