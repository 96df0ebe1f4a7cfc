// Host launchers for the gfx950 kernels (defined in kernels.hip; the fused
// block's launcher in block.hip). All launch on the given stream and return the
// launch status.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <string>

#include "conv_args.h"

namespace arthip {

// Compute units of the current device (queried once per device, thread-safe;
// 256 when unknown).
int cu_count();
// Multiply-shift constants for dividing uniform values < 2^31 by d on the GPU.
FastDiv make_fastdiv(uint32_t d);

// Largest channel counts the register-resident Winograd kernel is built for.
int winograd_max_kc();  // input channels <= 32 * winograd_max_kc()
int winograd_max_m();   // output channels

hipError_t launch_winograd(WinoArgs a, hipStream_t s);
hipError_t launch_direct(DirectArgs a, hipStream_t s);
// Fused residual block (winograd_block): C = M = 64, act2 none, act1 none /
// ReLU / SiLU, 0-2 residual inputs. block_eligible says whether a block of this
// geometry runs fused; launch_block refuses what it does not accept.
bool block_eligible(int C, int M, int act1, int act2, int64_t N, int64_t H, int64_t W);
hipError_t launch_block(BlockArgs a, hipStream_t s);
// A lone 64 -> 64 conv (bias, activation, no residual input) on the
// row-Winograd pipe (rowpipe.hip): padded NHWC fp16 in and out, or the NCHW
// fp16 boundary layout on the input (io bit 0) and / or output (io bit 1)
// side; rowpipe_eligible says whether it takes the shape.
bool rowpipe_eligible(int C, int M, int nskip, int act, int64_t N, int64_t H, int64_t W,
                      int io);
hipError_t launch_rowpipe(StripArgs a, int act, int io, hipStream_t s);
// A lone 96 -> 96 conv (bias, activation, at most one residual input; padded
// NHWC fp16 in and out) on the row-Winograd pipe (rowpipe96.hip);
// rowpipe96_eligible says whether it takes the shape.
bool rowpipe96_eligible(int C, int M, int nskip, int act, int64_t N, int64_t H, int64_t W,
                        int io);
hipError_t launch_rowpipe96(StripArgs a, int act, hipStream_t s);
hipError_t launch_eltwise(EltArgs a, bool binary, hipStream_t s);
hipError_t launch_dts(DtsArgs a, hipStream_t s);
hipError_t launch_input_convert(IoArgs a, hipStream_t s);
hipError_t launch_output_convert(IoArgs a, hipStream_t s);
hipError_t launch_plane_convert(PlaneArgs a, hipStream_t s);
// Fills the interior of a padded NHWC fp16 buffer holding an N x H x W x C
// tensor with `pattern` (diagnostics); the border keeps its zeros.
hipError_t launch_poison(void* buf, int32_t N, int32_t H, int32_t W, int32_t C, uint16_t pattern,
                         hipStream_t s);
// Zeroes everything of a padded NHWC fp16 buffer holding an N x H x W x C
// tensor except the interior: the border rows and columns (and the extra
// row / column of an odd H / W) that the convs read as zero padding.
hipError_t launch_zero_border(void* buf, int32_t N, int32_t H, int32_t W, int32_t C,
                              hipStream_t s);

// While alive (and `on`), this thread's stream-capture mode is relaxed, so
// that the library's own calls that are not stream work (hipEventQuery of work
// recorded outside a capture, hipFuncSetAttribute) do not invalidate a
// caller's global-mode capture; the kernels launched on the capturing stream
// are captured as in any mode. The previous mode is restored on destruction.
class RelaxedCaptureMode {
 public:
  explicit RelaxedCaptureMode(bool on) : on_(on) {
    if (on_ && hipThreadExchangeStreamCaptureMode(&mode_) != hipSuccess) on_ = false;
  }
  ~RelaxedCaptureMode() {
    if (on_) (void)hipThreadExchangeStreamCaptureMode(&mode_);
  }
  RelaxedCaptureMode(const RelaxedCaptureMode&) = delete;
  RelaxedCaptureMode& operator=(const RelaxedCaptureMode&) = delete;

 private:
  bool on_;
  hipStreamCaptureMode mode_ = hipStreamCaptureModeRelaxed;
};

// The no-allocation entry point's scratch: a file-scope device array of this
// many bytes, one copy on every GPU the library's code is loaded on, held until
// the process ends. scratch_setup resolves its address on `device` (which must
// be the calling thread's current device) and creates the event that orders
// its users; once per device, at engine set-up, so that the entry point's own
// calls create nothing.
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(256) << 20;
bool scratch_setup(int device, std::string& error);

// One call's use of a device's scratch, for every engine handle on that
// device. Begin takes the device's scratch lock (held until the object goes
// away) and orders stream s after the previous use when that was on another
// stream; on a capturing stream, which cannot wait on an event recorded
// outside the capture, the previous use must be over already, or Begin fails.
// End records the use's completion on s (not under capture: a captured use
// runs at each replay, which the caller orders).
class ScratchUse {
 public:
  ScratchUse() = default;
  ScratchUse(const ScratchUse&) = delete;
  ScratchUse& operator=(const ScratchUse&) = delete;
  ~ScratchUse();
  bool Begin(int device, hipStream_t s, bool capturing, void** ptr, std::string& error);
  bool End(std::string& error);

 private:
  void* dev_ = nullptr;
  bool locked_ = false;
  bool capturing_ = false;
  hipStream_t stream_ = nullptr;
};

}  // namespace arthip
