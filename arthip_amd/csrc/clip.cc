#include "clip.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>

#include "launch.h"
#include "onnx.h"

namespace arthip {

namespace {

std::string vs_error(const std::string& what) { return "hip.Model: " + what; }

int sample_kind(const VideoFormat& f) {
  if (f.sample_type == kStInteger) return f.bits_per_sample == 8 ? kSampleU8 : kSampleU16;
  return f.bits_per_sample == 16 ? kSampleF16 : kSampleF32;
}

size_t kind_bytes(int kind) {
  switch (kind) {
    case kSampleU8: return 1;
    case kSampleF32: return 4;
    default: return 2;
  }
}

// The VapourSynth loader's own checks before the engine sees the model
// (src/vapoursynth/onnx_utils.cpp:95-124 with specifyShape 29-75): one graph
// input and one output, both 4-D.
bool load_network(const ClipModelArgs& args, std::vector<uint8_t>& bytes, std::string& error) {
  if (!args.network_bytes.empty()) {
    bytes = args.network_bytes;
  } else {
    FILE* f = std::fopen(args.network_path.c_str(), "rb");
    if (!f) {
      error = "open " + args.network_path + " failed";
      return false;
    }
    bytes.clear();
    uint8_t chunk[1 << 16];
    size_t n;
    while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) bytes.insert(bytes.end(), chunk, chunk + n);
    std::fclose(f);
  }
  onnx::Model m;
  std::string perr;
  if (!onnx::ParseModel(bytes.data(), bytes.size(), m, perr)) {
    error = args.network_bytes.empty() ? "parse " + args.network_path + " failed"
                                       : std::string("parse onnx serialization failed");
    return false;
  }
  // Older IR versions list initializers among the graph inputs.
  size_t n_inputs = 0;
  const onnx::ValueInfo* gin = nullptr;
  for (const auto& vi : m.graph.inputs) {
    bool is_init = false;
    for (const auto& t : m.graph.initializers)
      if (t.name == vi.name) is_init = true;
    if (!is_init) {
      ++n_inputs;
      gin = &vi;
    }
  }
  if (n_inputs != 1) {
    error = "graph must has a single input";
    return false;
  }
  if (m.graph.outputs.size() != 1) {
    error = "graph must has a single output";
    return false;
  }
  if (gin->has_shape && gin->dims.size() != 4) {
    error = "input dimension must be 4";
    return false;
  }
  const onnx::ValueInfo& gout = m.graph.outputs[0];
  if (gout.has_shape && gout.dims.size() != 4) {
    error = "output dimsion must be 4";
    return false;
  }
  return true;
}

}  // namespace

namespace {

bool grow_dev(void*& p, size_t& cap, size_t need, std::string& error) {
  if (need <= cap) return true;
  if (p) hipFree(p);
  p = nullptr;
  cap = 0;
  const hipError_t e = hipMalloc(&p, need);
  if (e != hipSuccess) {
    p = nullptr;
    error = std::string("hipMalloc failed: ") + hipGetErrorString(e);
    return false;
  }
  cap = need;
  return true;
}

bool grow_host(void*& p, size_t& cap, size_t need, std::string& error) {
  if (need <= cap) return true;
  if (p) hipHostFree(p);
  p = nullptr;
  cap = 0;
  const hipError_t e = hipHostMalloc(&p, need, hipHostMallocDefault);
  if (e != hipSuccess) {
    p = nullptr;
    error = std::string("hipHostMalloc failed: ") + hipGetErrorString(e);
    return false;
  }
  cap = need;
  return true;
}

}  // namespace

// The staging of one frame in flight: raw plane samples (pinned host +
// device), the engine's boundary input and output, the integer output, the
// pinned download, and the event that marks the download done.
struct ClipModel::Io {
  std::mutex mu;  // held for a whole frame
  void* raw_host = nullptr;
  void* raw_dev = nullptr;
  void* in_dev = nullptr;
  void* out_dev = nullptr;
  void* out_int_dev = nullptr;
  void* out_host = nullptr;
  size_t raw_host_cap = 0, raw_dev_cap = 0, in_cap = 0, out_cap = 0, out_int_cap = 0,
         out_host_cap = 0;
  // Upload landed / kernels done / download done.
  hipEvent_t up = nullptr, comp = nullptr, done = nullptr;

  ~Io() {
    if (done) hipEventSynchronize(done);
    for (hipEvent_t ev : {up, comp, done})
      if (ev) hipEventDestroy(ev);
    if (raw_host) hipHostFree(raw_host);
    if (out_host) hipHostFree(out_host);
    for (void* p : {raw_dev, in_dev, out_dev, out_int_dev})
      if (p) hipFree(p);
  }
};

// Upload and download streams shared by every engine of the pool: PCIe is one
// resource, and one kernel stream per engine plus these two stays within the
// process's hardware queues (more streams than queues share queues and
// serialize).
struct ClipModel::CopyStreams {
  std::mutex mu;  // creation
  hipStream_t up = nullptr, down = nullptr;  // host -> device, device -> host

  ~CopyStreams() {
    for (hipStream_t st : {up, down})
      if (st) hipStreamSynchronize(st);
    for (hipStream_t st : {up, down})
      if (st) hipStreamDestroy(st);
  }
};

// One engine of the pool with its kernel stream and two staging sets. The
// engine lock covers only the enqueue of a frame's device work, and uploads and
// downloads run on the copy streams (ordered against the kernels by events), so
// one frame's host copies, wait and PCIe transfers overlap the next frame's
// kernels: with one engine and several callers, the frame time is the kernels'.
struct ClipModel::Slot {
  std::unique_ptr<Engine> eng;
  std::mutex mu;  // engine, stream, last shape; held while enqueuing
  hipStream_t stream = nullptr;              // kernels
  hipStream_t up = nullptr, down = nullptr;  // the pool's copy streams (not owned)
  int64_t last_shape[4] = {0, 0, 0, 0};
  Io io[2];
  // Profiling: an event after the engine's last launch (frames then run one at
  // a time per engine, so each frame's spans are read alone).
  hipEvent_t ev_run = nullptr;
  uint64_t frames = 0;

  ~Slot() {
    for (hipStream_t st : {up, stream, down})
      if (st) hipStreamSynchronize(st);
    if (ev_run) hipEventDestroy(ev_run);
    if (stream) hipStreamDestroy(stream);
  }
};

ClipModel::~ClipModel() = default;

int ClipModel::planes_written() const {
  if (flexible()) return out_channels_;
  return out_format_.color_family == kCfRGB ? 3 : 1;
}

std::unique_ptr<ClipModel> ClipModel::Create(const ClipModelArgs& args, int num_clips,
                                             const VideoFormat& fmt, int width, int height,
                                             std::string& error) {
  auto fail = [&](const std::string& msg) {
    error = vs_error(msg);
    return std::unique_ptr<ClipModel>();
  };
  if (num_clips != 1) return fail("expects exactly 1 input clip");
  std::unique_ptr<ClipModel> d(new ClipModel());
  d->flexible_prop_ = args.flexible_output_prop;

  // Static format checks (vs_hip.cpp:428-448).
  if (fmt.color_family != kCfGray && fmt.color_family != kCfYUV && fmt.color_family != kCfRGB)
    return fail("expects a gray, YUV or RGB clip");
  if (!((fmt.sample_type == kStInteger && (fmt.bits_per_sample == 8 || fmt.bits_per_sample == 16)) ||
        (fmt.sample_type == kStFloat && (fmt.bits_per_sample == 16 || fmt.bits_per_sample == 32))))
    return fail("expects 8/16-bit int or fp16/fp32 float input");
  if (fmt.sub_sampling_w != 0 || fmt.sub_sampling_h != 0)
    return fail("subsampled input (YUV420/YUV422) is not supported; convert to 4:4:4 first");

  // Options (vs_hip.cpp:454-464): an absent device_id / num_streams reads as 0,
  // num_streams < 1 means 1, fp16 defaults to true. Saturated to int.
  auto sat = [](int64_t v) {
    return static_cast<int>(v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : v));
  };
  d->device_ = args.has_device_id ? sat(args.device_id) : 0;
  {
    const char* e = std::getenv("VSHIP_PROFILE");
    d->profile_ = e != nullptr && e[0] == '1';
    const char* t = std::getenv("VSHIP_TRACE");
    d->trace_ = t != nullptr && t[0] == '1';
  }
  int num_streams = args.has_num_streams ? sat(args.num_streams) : 0;
  if (num_streams < 1) num_streams = 1;
  d->fp16_ = args.has_fp16 ? (args.fp16 != 0) : true;

  // Tiling arguments: only the no-tiling default is accepted (vs_hip.cpp:466-494).
  {
    const int64_t overlap_w = args.overlap.size() > 0 ? args.overlap[0] : 0;
    const int64_t overlap_h = args.overlap.size() > 1 ? args.overlap[1] : overlap_w;
    if (overlap_w < 0 || overlap_h < 0) return fail("\"overlap\" must be non-negative");
    if (overlap_w != 0 || overlap_h != 0)
      return fail("\"overlap\" is not supported: this filter always processes the whole frame in one tile");
    if (!args.tilesize.empty()) {
      const int64_t tile_w = args.tilesize[0];
      const int64_t tile_h = args.tilesize.size() > 1 ? args.tilesize[1] : tile_w;
      if (tile_w != width || tile_h != height)
        return fail("\"tilesize\" is not supported: this filter always processes the whole frame in one tile");
    }
  }

  std::vector<uint8_t> bytes;
  std::string lerr;
  if (!load_network(args, bytes, lerr)) return fail(lerr);

  // fp16=1: the fp32 -> fp16 model conversion, keeping fp32 IO only for an
  // fp32 clip (vs_hip.cpp:503-515).
  BuildOptions opts;
  opts.fp16 = d->fp16_;
  opts.keep_io_fp32 = fmt.sample_type == kStFloat && fmt.bits_per_sample == 32;

  d->copy_ = std::make_unique<CopyStreams>();
  for (int i = 0; i < num_streams; ++i) {
    auto s = std::make_unique<Slot>();
    s->eng = std::make_unique<Engine>(d->device_);
    std::string berr;
    if (!s->eng->Build(bytes.data(), bytes.size(), berr, opts)) return fail(berr);
    if (d->profile_) s->eng->SetProfiling(true);
    d->slots_.push_back(std::move(s));
  }
  Engine& e0 = *d->slots_[0]->eng;
  d->in_fp32_ = e0.InputFp32();
  d->out_fp32_ = e0.OutputFp32();
  d->in_channels_ = e0.InputChannels();
  if (d->in_channels_ < 1) d->in_channels_ = 1;

  // Plane count against the model's input channels (vs_hip.cpp:532-544).
  if (d->in_channels_ > 3)
    return fail("model requires " + std::to_string(d->in_channels_) +
                " input channels, but a clip provides at most 3 full-resolution planes");
  if (fmt.num_planes != d->in_channels_)
    return fail("clip has " + std::to_string(fmt.num_planes) + " plane(s) but the model expects " +
                std::to_string(d->in_channels_) + " input channel(s)");

  // Output clip (vs_hip.cpp:546-575): the probe's final channels (after a
  // trailing DepthToSpace) and scale; RGB for 3 channels without the flexible
  // protocol; float unless fp16=0 with an fp16 output; 32 bits for fp32 output.
  const int64_t probe_in[4] = {1, d->in_channels_, 64, 64};
  int64_t probe_out[4];
  if (!e0.OutputShape(probe_in, probe_out)) return fail("model shape probe failed");
  d->out_channels_ = static_cast<int>(probe_out[1]);
  if (d->out_channels_ < 1) d->out_channels_ = 1;
  const int scale_w = static_cast<int>(probe_out[3] / probe_in[3]);
  const int scale_h = static_cast<int>(probe_out[2] / probe_in[2]);
  d->scale_w_ = scale_w;
  d->scale_h_ = scale_h;
  d->out_width_ = width * scale_w;
  d->out_height_ = height * scale_h;
  VideoFormat& of = d->out_format_;
  of.color_family = (d->out_channels_ == 3 && d->flexible_prop_.empty()) ? kCfRGB : kCfGray;
  of.sample_type = (d->out_fp32_ || d->fp16_) ? kStFloat : kStInteger;
  of.bits_per_sample = d->out_fp32_ ? 32 : 16;
  of.sub_sampling_w = of.sub_sampling_h = 0;
  of.num_planes = of.color_family == kCfRGB ? 3 : 1;
  return d;
}

ClipModel::Slot& ClipModel::Acquire(std::unique_lock<std::mutex>& lock, Io*& io) {
  // Round-robin start (vs_hip.cpp:121-123), but take the first idle staging
  // set from there instead of queueing behind a busy engine.
  const unsigned n = static_cast<unsigned>(slots_.size());
  const unsigned start = next_.fetch_add(1);
  for (unsigned k = 0; k < 2 * n; ++k) {
    Slot& s = *slots_[(start + k) % n];
    Io& cand = s.io[((start + k) / n) & 1];
    std::unique_lock<std::mutex> l(cand.mu, std::try_to_lock);
    if (l.owns_lock()) {
      lock = std::move(l);
      io = &cand;
      return s;
    }
  }
  Slot& s = *slots_[start % n];
  io = &s.io[(start / n) & 1];
  lock = std::unique_lock<std::mutex>(io->mu);
  return s;
}

bool ClipModel::GetFrame(const VideoFormat& fmt, const int* plane_w, const int* plane_h,
                         const void* const* src, const ptrdiff_t* src_stride, void* const* dst,
                         const ptrdiff_t* dst_stride, int n_dst, std::string& error) {
  auto fail = [&](const std::string& msg) {
    error = vs_error(msg);
    return false;
  };
  if (fmt.num_planes < 1 || plane_w == nullptr || plane_h == nullptr || src == nullptr ||
      src_stride == nullptr)
    return fail("null or empty source frame");
  // Per-frame checks for variable-format clips (vs_hip.cpp:99-119).
  const int in_w = plane_w[0], in_h = plane_h[0];
  for (int p = 1; p < fmt.num_planes; ++p)
    if (plane_w[p] != in_w || plane_h[p] != in_h)
      return fail("subsampled input frame: every plane must have the luma plane's dimensions");
  const int in_c = fmt.num_planes;
  if (in_c != in_channels_ || in_c > 3)
    return fail("input clip plane count does not match the model's input channels");
  if (!((fmt.sample_type == kStInteger && (fmt.bits_per_sample == 8 || fmt.bits_per_sample == 16)) ||
        (fmt.sample_type == kStFloat && (fmt.bits_per_sample == 16 || fmt.bits_per_sample == 32))))
    return fail("expects 8/16-bit int or fp16/fp32 float input");
  if (in_w <= 0 || in_h <= 0) return fail("shape propagation failed");
  const size_t bps = kind_bytes(sample_kind(fmt));
  for (int p = 0; p < in_c; ++p)
    if (src[p] == nullptr || src_stride[p] < static_cast<ptrdiff_t>(in_w * bps))
      return fail("null source plane or stride shorter than a row");
  const int need = planes_written();
  if (dst == nullptr || dst_stride == nullptr || n_dst < need)
    return fail("expected " + std::to_string(need) + " destination plane(s), got " +
                std::to_string(n_dst));
  for (int c = 0; c < need; ++c)
    if (dst[c] == nullptr) return fail("null destination plane");

  std::unique_lock<std::mutex> lock;
  Io* io = nullptr;
  Slot& s = Acquire(lock, io);
  if (!trace_) return RunSlot(s, *io, fmt, in_c, in_w, in_h, src, src_stride, dst, dst_stride, error);
  int ei = 0;
  for (size_t q = 0; q < slots_.size(); ++q)
    if (slots_[q].get() == &s) ei = static_cast<int>(q);
  const unsigned long long n = frames_.fetch_add(1);
  auto now = [] {
    return (long long)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
  };
  std::fprintf(stderr, "[trace] enter eng=%d n=%llu t=%lld\n", ei, n, now());
  std::fflush(stderr);
  const bool ok = RunSlot(s, *io, fmt, in_c, in_w, in_h, src, src_stride, dst, dst_stride, error);
  std::fprintf(stderr, "[trace] leave eng=%d n=%llu t=%lld%s\n", ei, n, now(), ok ? "" : " failed");
  std::fflush(stderr);
  return ok;
}

bool ClipModel::RunSlot(Slot& s, Io& io, const VideoFormat& fmt, int in_c, int w, int h,
                        const void* const* src, const ptrdiff_t* src_stride, void* const* dst,
                        const ptrdiff_t* dst_stride, std::string& error) {
  auto fail = [&](const std::string& msg) {
    error = vs_error(msg);
    return false;
  };
  auto hip_fail = [&](const char* what, hipError_t e) {
    return fail(std::string(what) + ": " + hipGetErrorString(e));
  };
  Engine& eng = *s.eng;
  const int64_t in_shape[4] = {1, in_c, h, w};
  int64_t out_shape[4];
  if (!eng.OutputShape(in_shape, out_shape)) return fail("shape propagation failed");
  const int out_c = static_cast<int>(out_shape[1]);
  const int out_h = static_cast<int>(out_shape[2]);
  const int out_w = static_cast<int>(out_shape[3]);
  const int n_out = planes_written() < out_c ? planes_written() : out_c;

  const int src_kind = sample_kind(fmt);
  const int in_kind = in_fp32_ ? kSampleF32 : kSampleF16;
  const size_t in_px = static_cast<size_t>(w) * h;
  const size_t raw_row = static_cast<size_t>(w) * kind_bytes(src_kind);
  const size_t raw_bytes = raw_row * h * in_c;
  const size_t in_bytes = in_px * in_c * kind_bytes(in_kind);
  const size_t out_px = static_cast<size_t>(out_w) * out_h;
  const size_t out_bytes = out_px * out_c * (out_fp32_ ? 4 : 2);
  const bool int_out = out_format_.sample_type == kStInteger;
  // Only the channels written leave the GPU, as fp32, fp16 or u16 samples.
  const size_t obps = out_fp32_ ? 4 : 2;
  const size_t orow = static_cast<size_t>(out_w) * obps;
  const size_t dl_bytes = orow * out_h * n_out;
  const bool direct_in = src_kind == in_kind;  // samples already in the boundary type
  for (int c = 0; c < n_out; ++c)
    if (dst_stride[c] < static_cast<ptrdiff_t>(orow)) return fail("destination stride shorter than a row");

  hipError_t e = hipSetDevice(device_);
  if (e != hipSuccess) return hip_fail("hipSetDevice", e);
  std::string aerr;
  if (!grow_host(io.raw_host, io.raw_host_cap, raw_bytes, aerr) ||
      !grow_host(io.out_host, io.out_host_cap, dl_bytes, aerr))
    return fail(aerr);

  // Host: plane rows into pinned staging, plane-major, samples as they are.
  uint8_t* stage = static_cast<uint8_t*>(io.raw_host);
  for (int c = 0; c < in_c; ++c) {
    const uint8_t* base = static_cast<const uint8_t*>(src[c]);
    uint8_t* out = stage + static_cast<size_t>(c) * raw_row * h;
    if (src_stride[c] == static_cast<ptrdiff_t>(raw_row)) {
      std::memcpy(out, base, raw_row * h);
    } else {
      for (int y = 0; y < h; ++y)
        std::memcpy(out + static_cast<size_t>(y) * raw_row, base + static_cast<ptrdiff_t>(y) * src_stride[c],
                    raw_row);
    }
  }

  {
    // Device work of the frame, enqueued under the engine lock. With profiling
    // the lock covers the whole frame.
    std::unique_lock<std::mutex> elock(s.mu);
    // After a failure, work already queued may still read this staging set,
    // which the next caller may reuse: drain the stream before returning.
    auto drain = [&](bool r) {
      if (!r)
        for (hipStream_t st : {s.up, s.stream, s.down})
          if (st) (void)hipStreamSynchronize(st);
      return r;
    };
    // The same when the section is left by an exception (an allocation
    // failure): the caller reports it, and the staging set must be idle first.
    struct DrainOnThrow {
      const Slot& s;
      const int uncaught = std::uncaught_exceptions();
      ~DrainOnThrow() {
        if (std::uncaught_exceptions() > uncaught)
          for (hipStream_t st : {s.up, s.stream, s.down})
            if (st) (void)hipStreamSynchronize(st);
      }
    } drain_on_throw{s};
    if (s.up == nullptr) {
      std::lock_guard<std::mutex> g(copy_->mu);
      for (hipStream_t* st : {&copy_->up, &copy_->down})
        if (*st == nullptr && (e = hipStreamCreateWithFlags(st, hipStreamNonBlocking)) != hipSuccess) {
          *st = nullptr;
          return hip_fail("hipStreamCreate", e);
        }
      s.up = copy_->up;
      s.down = copy_->down;
    }
    if (s.stream == nullptr && (e = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking)) != hipSuccess) {
      s.stream = nullptr;
      return hip_fail("hipStreamCreate", e);
    }
    for (hipEvent_t* ev : {&io.up, &io.comp, &io.done})
      if (*ev == nullptr && (e = hipEventCreateWithFlags(ev, hipEventDisableTiming)) != hipSuccess) {
        *ev = nullptr;
        return hip_fail("hipEventCreate", e);
      }
    // A new frame shape re-plans the engine, which frees buffers that earlier
    // frames may still use: drain first.
    if (std::memcmp(s.last_shape, in_shape, sizeof in_shape) != 0) {
      for (hipStream_t st : {s.up, s.stream, s.down})
        if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail("HIP stream synchronize", e);
      std::memcpy(s.last_shape, in_shape, sizeof in_shape);
    }
    if (!grow_dev(io.in_dev, io.in_cap, in_bytes, aerr) ||
        (!direct_in && !grow_dev(io.raw_dev, io.raw_dev_cap, raw_bytes, aerr)) ||
        !grow_dev(io.out_dev, io.out_cap, out_bytes, aerr) ||
        (int_out && !grow_dev(io.out_int_dev, io.out_int_cap, dl_bytes, aerr)))
      return fail(aerr);
    void* upload_dst = direct_in ? io.in_dev : io.raw_dev;
    if ((e = hipMemcpyAsync(upload_dst, io.raw_host, raw_bytes, hipMemcpyHostToDevice, s.up)) != hipSuccess ||
        (e = hipEventRecord(io.up, s.up)) != hipSuccess ||
        (e = hipStreamWaitEvent(s.stream, io.up, 0)) != hipSuccess)
      return drain(hip_fail("HIP input upload", e));
    if (!direct_in) {
      PlaneArgs pa{io.raw_dev, io.in_dev, static_cast<int64_t>(in_px * in_c), src_kind, in_kind};
      if ((e = launch_plane_convert(pa, s.stream)) != hipSuccess) return drain(hip_fail("plane_convert", e));
    }
    std::string rerr;
    if (!eng.RunDevice(io.in_dev, in_shape, io.out_dev, s.stream, rerr)) return drain(fail(rerr));
    const bool prof = profile_ && (s.ev_run != nullptr || hipEventCreate(&s.ev_run) == hipSuccess);
    if (prof && (e = hipEventRecord(s.ev_run, s.stream)) != hipSuccess)
      return drain(hip_fail("HIP event record", e));
    const void* dl_src = io.out_dev;
    if (int_out) {
      PlaneArgs pa{io.out_dev, io.out_int_dev, static_cast<int64_t>(out_px * n_out), kSampleF16,
                   kSampleU16};
      if ((e = launch_plane_convert(pa, s.stream)) != hipSuccess) return drain(hip_fail("plane_convert", e));
      dl_src = io.out_int_dev;
    }
    if ((e = hipEventRecord(io.comp, s.stream)) != hipSuccess ||
        (e = hipStreamWaitEvent(s.down, io.comp, 0)) != hipSuccess ||
        (e = hipMemcpyAsync(io.out_host, dl_src, dl_bytes, hipMemcpyDeviceToHost, s.down)) != hipSuccess)
      return drain(hip_fail("HIP output download", e));
    if ((e = hipEventRecord(io.done, s.down)) != hipSuccess) return drain(hip_fail("HIP event record", e));
    if (prof) {
      if ((e = hipEventSynchronize(io.done)) != hipSuccess) return drain(hip_fail("HIP event synchronize", e));
      std::vector<Engine::StepProfile> steps;
      std::string perr;
      if (!eng.ProfileRead(steps, perr)) return drain(fail(perr));
      const uint64_t f = ++s.frames;
      if (f <= 3 || f % 128 == 0) {
        // io.done has no timing: the transfer span ends at a timed event.
        hipEvent_t end = nullptr;
        float xfer = 0.0f;
        if (hipEventCreate(&end) == hipSuccess) {
          if (hipEventRecord(end, s.down) == hipSuccess && hipEventSynchronize(end) == hipSuccess)
            hipEventElapsedTime(&xfer, s.ev_run, end);
          hipEventDestroy(end);
        }
        std::fprintf(stderr, "[vship-prof] frame %llu\n", static_cast<unsigned long long>(f));
        for (size_t i = 0; i < steps.size(); ++i)
          std::fprintf(stderr, "[vship-prof] op%-2zu %s %8.3f ms\n", i, steps[i].name.c_str(),
                       steps[i].total_ms);
        std::fprintf(stderr, "[vship-prof] output-convert+download %8.3f ms\n", xfer);
        std::fflush(stderr);
      }
    }
  }
  // Outside the engine lock: wait for this frame's download, copy it out.
  if ((e = hipEventSynchronize(io.done)) != hipSuccess) return hip_fail("HIP output download", e);

  // Host: rows out of pinned staging into the destination planes.
  const uint8_t* ost = static_cast<const uint8_t*>(io.out_host);
  for (int c = 0; c < n_out; ++c) {
    const uint8_t* from = ost + static_cast<size_t>(c) * orow * out_h;
    uint8_t* base = static_cast<uint8_t*>(dst[c]);
    if (dst_stride[c] == static_cast<ptrdiff_t>(orow)) {
      std::memcpy(base, from, orow * out_h);
    } else {
      for (int y = 0; y < out_h; ++y)
        std::memcpy(base + static_cast<ptrdiff_t>(y) * dst_stride[c], from + static_cast<size_t>(y) * orow, orow);
    }
  }
  return true;
}

}  // namespace arthip
