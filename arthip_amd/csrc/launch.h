// Host launchers for the gfx950 kernels (defined in kernels.hip; the fused
// block's launcher in block.hip). All launch on the given stream and return the
// launch status.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <string>

#include "conv_args.h"

namespace arthip {

// Compute units of the current device (queried once; 256 when unknown).
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

// The no-allocation entry point's scratch: a file-scope device array of this
// many bytes, one copy on every GPU the library's code is loaded on, held until
// the process ends. scratch_address gives its address on `device`, which must
// be the calling thread's current device (resolved once per device).
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(256) << 20;
bool scratch_address(int device, void** ptr, std::string& error);

}  // namespace arthip
