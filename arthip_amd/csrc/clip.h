// The VapourSynth filter core: hip.Model (src/vapoursynth/vs_hip.cpp) with the
// VapourSynth types replaced by plain formats, plane pointers and strides, so
// a VapourSynth adapter (VapourSynthPluginInit2 / createVideoFilter) reduces to
// argument marshalling and frame allocation around it.
//
// Create validates the clip format and the filter arguments with the
// reference's rules and error texts (vs_hip.cpp:401-591), loads the model,
// applies the load-time fp16 conversion and builds num_streams engines.
// GetFrame runs one frame on an idle staging set of the pool (two per engine:
// one frame's host copies overlap the next one's device work). Per frame the host only
// copies plane rows into pinned staging and back out: the samples cross PCIe
// in their own type (1 byte per 8-bit sample, not a float), and the scaling to
// [0, 1], the fp16 / fp32 rounding and the integer output conversion run on the
// GPU (plane_convert).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "engine.h"

namespace arthip {

// VapourSynth's VSColorFamily / VSSampleType numbering (VapourSynth4.h).
enum ColorFamily { kCfUndefined = 0, kCfGray = 1, kCfRGB = 2, kCfYUV = 3 };
enum SampleType { kStInteger = 0, kStFloat = 1 };

struct VideoFormat {
  int color_family = kCfUndefined;
  int sample_type = kStInteger;
  int bits_per_sample = 0;
  int sub_sampling_w = 0, sub_sampling_h = 0;
  int num_planes = 0;
};

// hip.Model's arguments (vs_hip.cpp:628-637). An absent optional is an empty
// vector / string, or has_* false.
struct ClipModelArgs {
  std::string network_path;
  std::vector<uint8_t> network_bytes;  // used instead of the path when non-empty
  bool has_device_id = false;
  int64_t device_id = 0;
  bool has_num_streams = false;
  int64_t num_streams = 1;
  bool has_fp16 = false;
  int64_t fp16 = 1;
  std::vector<int64_t> overlap, tilesize;
  std::string flexible_output_prop;
};

class ClipModel {
 public:
  // num_clips: elements of the "clips" argument. width / height: the clip's
  // (0 for a variable-size clip). Errors carry the "hip.Model: " prefix.
  static std::unique_ptr<ClipModel> Create(const ClipModelArgs& args, int num_clips,
                                           const VideoFormat& clip_format, int width, int height,
                                           std::string& error);
  ~ClipModel();

  // Output clip description (vs_hip.cpp:554-581).
  const VideoFormat& out_format() const { return out_format_; }
  int out_width() const { return out_width_; }
  int out_height() const { return out_height_; }
  int scale_w() const { return scale_w_; }
  int scale_h() const { return scale_h_; }
  int out_channels() const { return out_channels_; }  // "num_planes" of the flexible protocol
  bool flexible() const { return !flexible_prop_.empty(); }
  bool input_fp32() const { return in_fp32_; }
  bool output_fp32() const { return out_fp32_; }
  int num_streams() const { return static_cast<int>(slots_.size()); }

  // Output channels GetFrame writes: 3 for an RGB frame, every model channel
  // with the flexible protocol (dst[c] = channel c; the adapter writes dst[0]
  // into the frame and each channel into a MlrtFlexible<c> frame property),
  // else 1 (channel 0 into the gray frame).
  int planes_written() const;

  // One frame (vs_hip.cpp:77-385). plane_w / plane_h / src / src_stride have
  // fmt.num_planes entries; dst / dst_stride have n_dst >= planes_written()
  // entries, each a plane of out_width x out_height samples of out_format().
  // Safe to call from several threads: each call takes a free engine of the
  // pool (or waits for one).
  bool GetFrame(const VideoFormat& fmt, const int* plane_w, const int* plane_h,
                const void* const* src, const ptrdiff_t* src_stride, void* const* dst,
                const ptrdiff_t* dst_stride, int n_dst, std::string& error);

 private:
  struct Io;
  struct Slot;
  struct CopyStreams;
  ClipModel() = default;
  Slot& Acquire(std::unique_lock<std::mutex>& lock, Io*& io);
  bool RunSlot(Slot& s, Io& io, const VideoFormat& fmt, int in_c, int w, int h,
               const void* const* src, const ptrdiff_t* src_stride, void* const* dst,
               const ptrdiff_t* dst_stride, std::string& error);

  // Declared before slots_ so that the engines' work drains before the shared
  // copy streams are destroyed.
  std::unique_ptr<CopyStreams> copy_;
  std::vector<std::unique_ptr<Slot>> slots_;
  std::atomic<unsigned> next_{0};
  // VSHIP_PROFILE=1 at creation: per-launch GPU spans and the output
  // conversion + download span on stderr for the first three frames of each
  // engine and every 128th (hip_engine.cc:1409-1604).
  bool profile_ = false;
  // VSHIP_TRACE=1 at creation: "[trace] enter" / "[trace] leave" lines on
  // stderr around each frame's run, with the engine of the pool, the frame's
  // call number and a steady-clock timestamp in ns (vs_hip.cpp:239-246).
  bool trace_ = false;
  std::atomic<unsigned long long> frames_{0};
  int device_ = 0;
  bool fp16_ = true;
  bool in_fp32_ = false, out_fp32_ = false;
  int in_channels_ = 1, out_channels_ = 1;
  std::string flexible_prop_;
  VideoFormat out_format_{};
  int out_width_ = 0, out_height_ = 0;
  int scale_w_ = 1, scale_h_ = 1;
};

}  // namespace arthip
