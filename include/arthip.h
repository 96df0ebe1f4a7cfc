/*
 * arthip.h - C ABI of libarthip.so, the MI355X (gfx950) engine for
 * ArtCNN-style conv-chain upscalers (3x3 convs, ReLU/SiLU, residual adds,
 * DepthToSpace, Clip) stored as fp16 ONNX models.
 *
 * Plain C types only: pointers, sizes, error buffers. Return codes follow the
 * reference's test driver (tests/correctness/harness/engine_harness.cc:12-15):
 *   0 = ok, 1 = build / shape / argument failure, 2 = run failure.
 * Error text is copied NUL-terminated into (err, errlen) when given.
 */
#ifndef ARTHIP_H_
#define ARTHIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARTHIP_OK 0
#define ARTHIP_ERR_BUILD 1
#define ARTHIP_ERR_RUN 2

/* ------------------------------------------------------------------------ */
/* Engine handle                                                             */
/*                                                                           */
/* One engine = one compiled model on one device with its own HIP stream and */
/* mutex. It replaces vship::HipEngine (src/vapoursynth/hip_engine.h:88-188)  */
/* and onnxruntime::hip::HipGraph (src/onnxruntime-hip/hip_graph.h:113-167), */
/* which the VapourSynth plugin and the ONNX Runtime EP each drive.          */
/* Calls on one handle from several threads are serialized by that mutex (as */
/* HipGraph::Run's lock, hip_graph.cc:1212); destroy must not overlap any    */
/* other call on the handle. No entry point lets a C++ exception escape.     */
/* ------------------------------------------------------------------------ */

typedef struct arthip_engine arthip_engine;

/* Creates an engine bound to device_id (HipEngine::HipEngine,
 * hip_engine.h:90). No device work happens here or in build: the device is
 * selected and the stream created on the first run, which reports an invalid
 * device. */
int arthip_engine_create(int device_id, arthip_engine** out, char* err, int errlen);

void arthip_engine_destroy(arthip_engine* eng);

/* Parses, validates and fuses an ONNX model (HipEngine::Build,
 * hip_engine.h:92; hip_engine.cc:197-666). */
int arthip_engine_build_file(arthip_engine* eng, const char* path, char* err, int errlen);
int arthip_engine_build_bytes(arthip_engine* eng, const void* data, size_t size, char* err,
                              int errlen);

/* NCHW output shape for an NCHW input shape (HipEngine::GetOutputShape,
 * hip_engine.h:95-96). Returns 1 when shape propagation fails. */
int arthip_engine_output_shape(const arthip_engine* eng, const int64_t in_nchw[4],
                               int64_t out_nchw[4]);

/* Model IO description (InputIsFp32 / OutputIsFp32 / InputChannels /
 * OutputChannels, hip_engine.h:116-136). Any pointer may be NULL. */
int arthip_engine_io_info(const arthip_engine* eng, int* in_fp32, int* out_fp32,
                          int* in_channels, int* out_channels);

/* One frame from host memory to host memory (HipEngine::Run,
 * hip_engine.h:102-103): in_host is NCHW in the model's input dtype (fp16, or
 * fp32 when in_fp32), out_host receives NCHW in the output dtype; out_cap is
 * its size in bytes. Plans are cached per input shape. */
int arthip_engine_run(arthip_engine* eng, const void* in_host, const int64_t in_nchw[4],
                      void* out_host, size_t out_cap, char* err, int errlen);

/* The same with device-resident IO on a caller stream (NULL = the engine's
 * stream). No host copies and no host synchronisation: the caller orders its
 * own producers of in_dev and consumers of out_dev on that stream. Runs on
 * one handle share its intermediate buffers, so the engine orders each run
 * (run or run_device) after the previous one on the GPU, whatever streams
 * they were given (an event at the end of every run; the next run's stream
 * waits on it when the stream differs). The reference has no counterpart (its
 * Run always stages through host memory and serializes on its one stream,
 * hip_engine.cc:1282); this is the entry point for callers whose frames
 * already live in HBM. */
int arthip_engine_run_device(arthip_engine* eng, const void* in_dev, const int64_t in_nchw[4],
                             void* out_dev, void* stream, char* err, int errlen);

/* No counterpart in the reference: run_device for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results as
 * arthip_engine_run_device, but the intermediate activations live in the
 * library's scratch array, a file-scope device array of
 * ARTHIP_NOALLOC_SCRATCH_BYTES (256 MiB) that every GPU the library runs on
 * holds until the process ends; this call makes no hipMalloc, hipFree or other
 * allocating call.
 * - An input whose activations need more than the scratch holds is refused
 *   (return 2, with the bytes needed), before anything is enqueued. R8F64
 *   fits up to 960x540; R8F64 at 1920x1080 needs about 1.06 GB and must use
 *   run_device.
 * - The handle must have run once through arthip_engine_run or
 *   arthip_engine_run_device (any input size, e.g. a 2x2 warm-up): that run
 *   creates the engine's stream and uploads its weights. Otherwise return 2.
 * - Every call on one GPU shares that GPU's scratch, which keeps the last
 *   call's contents (each call clears the zero padding it needs). The calls
 *   of every handle on one GPU are ordered on the GPU by one event per GPU,
 *   created at engine set-up: a call whose stream differs from the last
 *   call's waits for it. Calls on one handle are also ordered after its
 *   run / run_device calls, like run_device.
 * - Under HIP graph capture (the stream is capturing): the call enqueues its
 *   launches into the graph. The handle's previous run and the GPU's previous
 *   scratch use must have finished (synchronize before capturing), since a
 *   captured call cannot wait on an event recorded outside the capture;
 *   otherwise return 2. Replays of the graph are not ordered against other
 *   calls on the handle or the scratch: the caller orders them (and must not
 *   replay while another call that uses the scratch is in flight).
 *   VSHIP_SYNC_EACH is refused under capture.
 * - Not profiled and not dumped (those create events and host buffers). */
#define ARTHIP_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int arthip_engine_run_device_noalloc(arthip_engine* eng, const void* in_dev,
                                     const int64_t in_nchw[4], void* out_dev, void* stream,
                                     char* err, int errlen);

/* Human-readable plan of the last built shape (op list, fusions, buffers). */
int arthip_engine_describe(const arthip_engine* eng, char* buf, int buflen);

/* Per-launch GPU timing (the reference's VSHIP_PROFILE per-op events,
 * hip_engine.cc:1409-1606): with profiling on, every launch of a run is
 * bracketed by HIP events on the launch stream. profile_read synchronizes
 * them and reports, per plan step, the summed milliseconds and launch count
 * since the previous read (arrays of max_steps; step names newline-separated
 * in names). Returns the number of plan steps, or a negative code. */
int arthip_engine_set_profiling(arthip_engine* eng, int on);
int arthip_engine_profile_read(arthip_engine* eng, int max_steps, double* total_ms,
                               int64_t* launches, char* names, int names_len, char* err,
                               int errlen);

/* Diagnostics: the reference's VSHIP_POISON (hip_engine.cc:1310-1323,
 * hip_graph.cc:1231-1248), VSHIP_SYNC_EACH (hip_graph.cc:1356-1365) and
 * VSHIP_DUMP (hip_engine.cc:1325-1349, 1509-1519). A new engine takes them
 * from those environment variables ("1", or a directory for VSHIP_DUMP);
 * set_debug replaces them.
 * - POISON: before each run, every internal activation's interior is filled
 *   with fp16 NaN (0x7E7E); the zero border of the padded layout stays. A
 *   read of a tensor no launch of the run has written turns into NaN.
 * - SYNC_EACH: the launch stream is synchronized after every launch and its
 *   status checked.
 * - DUMP: for the engine's first two runs, every launch's input buffers and
 *   output buffer are written to dump_dir/runR_opKK_inI.bin and
 *   runR_opKK_out.bin (raw bytes; internal activations in the padded NHWC
 *   fp16 layout of arthip_padded_dims, boundary tensors as given).
 * - UNFUSED (no environment switch): every conv runs as its own launch; by
 *   default a 64 -> 64 conv whose output only the next 64 -> 64 conv reads
 *   runs fused with it (arthip_conv3x3_block_f16_nhwc), which agrees with
 *   separate launches to fp16 rounding. Changing it drops the cached plans.
 * Host-side lines, written to the engine's log (stderr, or the file given to
 * arthip_engine_set_log):
 * - TRACE (VSHIP_TRACE=1; hip_engine.cc:1280-1298,1421-1425,1619): per run
 *   "[run] enter #R <entry> in=<ptr>", "[run] built #R" once the plan is
 *   ready, "[run] #R opK <step>" after each launch, then "[run] done #R
 *   out=<ptr>" or "[run] fail #R: <error>".
 * - HOST_PROFILE (HIP_PROFILE=1; hip_graph.cc:1213-1447): host time spans of
 *   each run. arthip_engine_run: "[hipprof] build= memin= launch=
 *   readback+wait=" and "[hipprof] memout= total=" (ms); the device entry
 *   points: "[hipprof] build= launch= total=" (enqueue only).
 * - DUMPOPS (HIP_DUMPOPS set to any value; hip_graph.cc:1366-1373): per launch
 *   "[dump] op K <step> in=<buf>(<ptr>,<MB>MB) ... out=<buf>(<ptr>,<MB>MB)",
 *   buffers by plan index, or input / output for the boundary tensors.
 * - PLAN (VSHIP_DEBUG=1; hip_engine.cc:1167-1184): each new plan's launch list,
 *   "[vship] plan for [N,C,H,W]: ..." and one "[vship] stepK" line per launch.
 * Returns 1 on an unknown flag or DUMP without a directory. */
#define ARTHIP_DEBUG_POISON 1
#define ARTHIP_DEBUG_SYNC_EACH 2
#define ARTHIP_DEBUG_DUMP 4
#define ARTHIP_DEBUG_UNFUSED 8
#define ARTHIP_DEBUG_TRACE 16
#define ARTHIP_DEBUG_HOST_PROFILE 32
#define ARTHIP_DEBUG_DUMPOPS 64
#define ARTHIP_DEBUG_PLAN 128
int arthip_engine_set_debug(arthip_engine* eng, int flags, const char* dump_dir);
int arthip_engine_get_debug(const arthip_engine* eng, int* flags);
/* Log of the TRACE / HOST_PROFILE / DUMPOPS / PLAN lines: appended to the file
 * at path, or stderr for NULL or "" (the default, as the reference writes
 * them). Returns 1 if the file cannot be opened (the log is unchanged). */
int arthip_engine_set_log(arthip_engine* eng, const char* path, char* err, int errlen);

/* ------------------------------------------------------------------------ */
/* ONNX Runtime execution provider: partitioning and compile                  */
/* ------------------------------------------------------------------------ */

/* GetCapability (src/onnxruntime-hip/hip_execution_provider.cc:181-335 with
 * IsNodeSupported 22-177): the maximal runs of consecutive supported nodes
 * of a serialized model, keeping only runs with one activation input and one
 * needed output. Run r is nodes[run_start[r] .. run_start[r+1]) (node indices
 * in graph order). device_id >= 0 first initializes that device and claims
 * nothing (*n_runs = 0, return 0) when it cannot (the reference's refusal after
 * a failed context init); device_id < 0 skips the device. Returns 1 on a
 * malformed model or when max_runs + 1 / max_nodes entries do not suffice (then
 * *n_runs and *n_nodes still give the sizes needed). Supported beyond the
 * reference: Relu. Refused beyond it: a Conv over the engine's channel limits. */
int arthip_ep_get_capability(const void* model, size_t size, int device_id, int* n_runs,
                             int* run_start, int max_runs, int* n_nodes, int* nodes,
                             int max_nodes, char* err, int errlen);

/* The fused node's MetaDef for a run (hip_execution_provider.cc:244-330): its
 * external activations (the claimed runs have exactly one, input 0), the
 * initializers its nodes read (the inputs after it) and the outputs needed
 * outside it, each deduplicated in first-seen order. Names are written
 * NUL-separated into the three buffers, with their counts; returns 1 when the
 * node list is invalid or a buffer is too small. */
int arthip_ep_run_boundary(const void* model, size_t size, const int* nodes, int n_nodes,
                           char* activations, int activations_len, int* n_activations,
                           char* constants, int constants_len, int* n_constants, char* outputs,
                           int outputs_len, int* n_outputs, char* err, int errlen);

/* The key of each listed node, for mapping a run onto the caller's own graph
 * (IndexedSubGraph::Nodes() takes ORT NodeIndex values,
 * hip_execution_provider.cc:303-306): the node's first non-empty output name,
 * NUL-separated in node order. ONNX gives every tensor name one producer, so
 * a key names the same node in the caller's graph whatever its node order;
 * node indices are positions in the serialized model only. Returns 1 for an
 * index outside the graph, a node without outputs or a buffer too small. */
int arthip_ep_node_keys(const void* model, size_t size, const int* nodes, int n_nodes,
                        char* keys, int keys_len, char* err, int errlen);

/* Compile for one claimed run (hip_execution_provider.cc:337-357): builds the
 * engine from the run's nodes of the serialized model, with the run's single
 * activation as input 0 and its single output as output 0. The reference
 * compiles the fused node's filtered graph; serialized on its own (its nodes,
 * the run's inputs including the initializers, their initializers, the run's
 * output), that graph is such a model with nodes 0 .. n-1. */
int arthip_engine_build_subgraph(arthip_engine* eng, const void* model, size_t size,
                                 const int* nodes, int n_nodes, char* err, int errlen);

/* ------------------------------------------------------------------------ */
/* Test-driver ABI: same names, arguments and return codes as the reference's */
/* ctypes driver (tests/correctness/harness/engine_harness.cc:56-210). Each   */
/* call builds a fresh engine from a model file.                              */
/* ------------------------------------------------------------------------ */

int engine_device_count(int* count);

int engine_probe(const char* model_path, int N, int H, int W, int C, int device, char* err,
                 int errlen, int* in_fp32, int* out_fp32, int* cin, int* cout,
                 int64_t* out_shape, int* out_rank);

int engine_run(const char* model_path, int N, int H, int W, int C, int device,
               const void* input, size_t input_bytes, void* out, size_t cap,
               size_t* out_bytes, int* out_fp32, int64_t* out_shape, int* out_rank, char* err,
               int errlen);

int engine_alloc_failure_then_run(const char* model_path, int N, int bigH, int bigW, int C,
                                  int device, const void* recovery_input,
                                  size_t recovery_input_bytes, void* out, size_t cap,
                                  size_t* out_bytes, int* out_fp32, int64_t* out_shape,
                                  int* out_rank, char* failerr, int failerrlen, char* runerr,
                                  int runerrlen);

/* ------------------------------------------------------------------------ */
/* VapourSynth filter core: hip.Model, Version and DeviceProperties          */
/* (src/vapoursynth/vs_hip.cpp:401-591, 77-385, 597-641) with VapourSynth's   */
/* types replaced by plain formats and plane pointers. A VapourSynth adapter  */
/* maps the filter's VSMap arguments into arthip_vs_model_args, calls         */
/* arthip_vs_model_create from its create callback and                        */
/* arthip_vs_model_get_frame from getFrame (fmParallel-safe). Error texts     */
/* carry the reference's "hip.Model: " prefix and wording.                    */
/* ------------------------------------------------------------------------ */

typedef struct arthip_vs_model arthip_vs_model;

/* VSVideoFormat's fields that the filter reads. color_family uses
 * VSColorFamily (0 undefined, 1 gray, 2 RGB, 3 YUV); sample_type uses
 * VSSampleType (0 integer, 1 float). */
typedef struct arthip_vs_format {
  int color_family;
  int sample_type;
  int bits_per_sample;
  int sub_sampling_w;
  int sub_sampling_h;
  int num_planes;
} arthip_vs_format;

/* hip.Model's arguments (vs_hip.cpp:628-637). has_* = 0 marks an absent
 * optional; overlap / tilesize with length 0 and a NULL or empty
 * flexible_output_prop are absent. network_data / network_size, when
 * network_size > 0, replace network_path with serialized model bytes. */
typedef struct arthip_vs_model_args {
  const char* network_path;
  const void* network_data;
  size_t network_size;
  int has_device_id;
  int64_t device_id;
  int has_num_streams;
  int64_t num_streams;
  int has_fp16;
  int64_t fp16;
  const int64_t* overlap;
  int overlap_len;
  const int64_t* tilesize;
  int tilesize_len;
  const char* flexible_output_prop;
} arthip_vs_model_args;

/* The output clip (vs_hip.cpp:554-581). num_planes is the model's final
 * output channel count (the flexible protocol's "num_planes");
 * planes_written is how many destination planes a frame call fills: 3 for an
 * RGB output, num_planes with the flexible protocol (plane c = channel c: the
 * adapter stores plane 0 in the frame and each plane as MlrtFlexible<c>), else
 * 1. in_fp32 / out_fp32 give the engine's boundary types after the load-time
 * fp16 conversion. A frame of w x h comes out as (w * scale_w) x (h * scale_h). */
typedef struct arthip_vs_model_info {
  arthip_vs_format format;
  int width;
  int height;
  int num_planes;
  int planes_written;
  int flexible;
  int in_fp32;
  int out_fp32;
  int num_streams;
  int scale_w;
  int scale_h;
} arthip_vs_model_info;

/* hipCreate (vs_hip.cpp:401-591): validates the clip format and the
 * arguments, loads the model (fp16 != 0, the default, applies the fp32 ->
 * fp16 model conversion), builds num_streams engines and describes the output
 * clip. width / height are the clip's. No device work happens here. Returns 1
 * with the error text on any refusal. */
int arthip_vs_model_create(const arthip_vs_model_args* args, int num_clips,
                           const arthip_vs_format* clip_format, int width, int height,
                           arthip_vs_model** out, arthip_vs_model_info* info, char* err,
                           int errlen);

/* hipGetFrame (vs_hip.cpp:77-385): one frame. fmt is the frame's format;
 * plane_w / plane_h / src / src_stride (bytes) have fmt->num_planes entries;
 * dst / dst_stride have n_dst >= planes_written entries, each an
 * info.width x info.height plane of info.format samples. Thread-safe; each
 * call runs on an idle engine of the pool, or waits for one. Returns 2 on
 * failure. */
int arthip_vs_model_get_frame(arthip_vs_model* model, const arthip_vs_format* fmt,
                              const int* plane_w, const int* plane_h, const void* const* src,
                              const ptrdiff_t* src_stride, void* const* dst,
                              const ptrdiff_t* dst_stride, int n_dst, char* err, int errlen);

void arthip_vs_model_destroy(arthip_vs_model* model);

/* hip.Version (vs_hip.cpp:597-603): the library version and, when the HIP
 * runtime answers, the device count (else *device_count = -1). */
int arthip_vs_version(char* version, int len, int* device_count);

/* hip.DeviceProperties (vs_hip.cpp:605-617). Returns 1 with
 * "hipDeviceProperties: failed to query device" when the query fails. */
int arthip_vs_device_properties(int device_id, char* name, int namelen, int64_t* pci_device_id,
                                int64_t* clock_rate, int64_t* global_memory, char* err,
                                int errlen);

/* ------------------------------------------------------------------------ */
/* Kernel-level entry points (one fused conv on device buffers)              */
/* ------------------------------------------------------------------------ */

/* Sizes of the packed filter buffer (in fp16 elements) and of the padded
 * fp32 bias buffer for a 3x3 conv with C inputs and M outputs. */
size_t arthip_conv3x3_packed_halfs(int M, int C);
size_t arthip_conv3x3_bias_len(int M);

/* Host-side filter transform, done once per layer: the Winograd
 * U = G g G^T for C > 1 (hip_engine.cc:972-1018), a tap relayout for C == 1
 * (hip_engine.cc:925-971). w_oihw holds fp16 bits [M][C][3][3]; bias holds M
 * fp16 values or is NULL. Outputs go to host buffers of the sizes above. */
int arthip_conv3x3_pack(const uint16_t* w_oihw, const uint16_t* bias, int M, int C,
                        uint16_t* packed, size_t packed_cap, float* bias_out, size_t bias_cap);

/* Internal activation layout used by the kernel-level entry points: NHWC fp16
 * with a zero border, [N][Hp][Wp][C] with Hp = 2*ceil(H/2) + 2 and
 * Wp = 2*ceil(W/2) + 2; pixel (h, w) lives at row h + 1, column w + 1. The
 * border must be zero (allocate zero-filled) and is never written. */
int arthip_padded_dims(int H, int W, int* Hp, int* Wp);

/* out = skip1 + skip0 + act(conv3x3(in) + bias) on padded NHWC fp16 device
 * buffers ([N][Hp][Wp][C] -> [N][Hp][Wp][M]); SAME padding, stride 1. act: 0
 * none, 1 ReLU, 2 SiLU. skip0/skip1: padded [N][Hp][Wp][M] or NULL. The fused
 * form of the reference's winograd_conv / direct_conv launches
 * (src/common/hip_kernels.h:143-483). stream may be NULL. */
int arthip_conv3x3_f16_nhwc(const void* in, const void* packed, const float* bias, int act,
                            const void* skip0, const void* skip1, void* out, int N, int H, int W,
                            int C, int M, void* stream);

/* A residual block of two fused 3x3 convs, C = M = 64:
 *   out = skip1 + skip0 + conv3x3_2(act1(conv3x3_1(in) + bias1)) + bias2
 * on padded NHWC fp16 device buffers of one geometry; the intermediate tensor
 * never leaves the chip. The fused form of the reference's two winograd_conv
 * launches with the residual Add fused into the second
 * (src/common/hip_kernels.h:143-396; hip_graph.cc:510-540). The intermediate
 * is computed with Winograd tiles at odd pixel offsets, so the result agrees
 * with two arthip_conv3x3_f16_nhwc calls to fp16 rounding (same error against
 * an exact reference), not bit for bit; it is bit-stable. packed1 / bias1 and packed2 /
 * bias2 come from arthip_conv3x3_pack. act1: 0 none, 1 ReLU, 2 SiLU. skip1
 * only with skip0; out must not alias in or a skip. The output stores carry
 * the non-temporal hint (an engine plan uses plain ones when the next launch
 * reads the output from HBM and it fits the last-level cache). Returns 1 for
 * other channel counts or a padded image of 2 GiB or more. */
int arthip_conv3x3_block_f16_nhwc(const void* in, const void* packed1, const float* bias1,
                                  int act1, const void* packed2, const float* bias2,
                                  const void* skip0, const void* skip1, void* out, int N, int H,
                                  int W, int C, void* stream);

/* Largest (C, M) the conv kernels accept. */
int arthip_conv3x3_limits(int* max_c, int* max_m);

/* ------------------------------------------------------------------------ */
/* Helpers                                                                   */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 round-to-nearest-even conversions
 * (HipEngine::FloatToHalfBitsRNE / HalfBitsToFloat, hip_engine.h:108-109). */
uint16_t arthip_f32_to_f16(float f);
float arthip_f16_to_f32(uint16_t h);

/* fp32 -> fp16 with the load-time model converter's rounding
 * (src/vapoursynth/convert_float_to_float16.cpp:158-186), which the
 * VapourSynth filter applies to fp32 initializers with fp16=1: nearest even,
 * but |f| < 2^-14 becomes a signed zero and NaN a signed inf. */
uint16_t arthip_f32_to_f16_no_subnormals(float f);

/* Thread-local text of the last failure of a kernel-level call. */
const char* arthip_last_error(void);

const char* arthip_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ARTHIP_H_ */
