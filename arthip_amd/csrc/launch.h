// Host launchers for the gfx950 kernels (defined in kernels.hip). All launch
// on the given stream and return the launch status.
#pragma once

#include <hip/hip_runtime.h>

#include "conv_args.h"

namespace arthip {

// Largest channel counts the register-resident Winograd kernel is built for.
int winograd_max_kc();  // input channels <= 32 * winograd_max_kc()
int winograd_max_m();   // output channels

hipError_t launch_winograd(WinoArgs a, hipStream_t s);
hipError_t launch_direct(DirectArgs a, hipStream_t s);
hipError_t launch_eltwise(EltArgs a, bool binary, hipStream_t s);
hipError_t launch_dts(DtsArgs a, hipStream_t s);
hipError_t launch_input_convert(IoArgs a, hipStream_t s);
hipError_t launch_output_convert(IoArgs a, hipStream_t s);
hipError_t launch_plane_convert(PlaneArgs a, hipStream_t s);
// Fills the interior of a padded NHWC fp16 buffer holding an N x H x W x C
// tensor with `pattern` (diagnostics); the border keeps its zeros.
hipError_t launch_poison(void* buf, int32_t N, int32_t H, int32_t W, int32_t C, uint16_t pattern,
                         hipStream_t s);

}  // namespace arthip
