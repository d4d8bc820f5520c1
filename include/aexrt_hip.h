/*
 * aexrt_hip.h -- C ABI of libaexrt_hip.so, the MI355X (gfx950) backend of the
 * AEXRT W8A8 convolution path.
 *
 * Conventions follow the reference's native/aexrt.h: opaque handles, int
 * return 1 = ok / 0 = failure, a NULL handle on failed creation, and a
 * diagnostic string from aexrt_hip_get_last_error() (per model:
 * aexrt_yolo_get_last_error).  Out-structs carry struct_size.  No function
 * takes a PyTorch type; device memory is passed as plain pointers.
 *
 * Two layers:
 *   1. op-level entry points on device pointers and a hipStream_t (passed as
 *      void*), one per hot-path kernel: amax, quantize, int8 / fp16 / Winograd
 *      convolution, and the weight repack they consume;
 *   2. the model-level API of aexrt.h (device, .aexrt engine load, run,
 *      errors, timing, conv plan inspection/override), executing the plan on
 *      HIP kernels with the whole run captured in a HIP graph.
 */
#ifndef AEXRT_HIP_H_
#define AEXRT_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* Shared types (same field order as native/aexrt.h)                       */
/* ---------------------------------------------------------------------- */

/* native/aexrt.h:98-115 AexrtConv2DDesc; the 16-u32 replay conv params
 * (src/aexrt/yolo.py:929-939). */
typedef struct AexrtConv2DDesc {
    uint32_t batch;
    uint32_t in_channels;
    uint32_t in_h;
    uint32_t in_w;
    uint32_t out_channels;
    uint32_t out_h;
    uint32_t out_w;
    uint32_t kernel_h;
    uint32_t kernel_w;
    uint32_t stride_h;
    uint32_t stride_w;
    uint32_t pad_top;
    uint32_t pad_left;
    uint32_t dilation_h;
    uint32_t dilation_w;
    uint32_t groups;
} AexrtConv2DDesc;

/* native/aexrt.h:20-27 */
typedef struct AexrtYoloDetection {
    float x1;
    float y1;
    float x2;
    float y2;
    float score;
    float class_id;
} AexrtYoloDetection;

/* An NHWC activation view on the device.  Element (n, h, w, c) of the view is
 * data[n * n_stride + (h * W + w) * c_stride + c] (elements of the view's
 * dtype).  amax_slots, when non-NULL, holds one uint32 per 16 channels of
 * the view: the bit pattern of max|x| over that channel group (all n, h, w).
 * The slot array may be striped: amax_stripes copies (0 counts as 1), copy s
 * at amax_slots + s * amax_stripe_stride.  Producers fold each workgroup's
 * maxima into one copy (spreading the atomics of thousands of workgroups
 * over several cache lines); readers take the max over all copies.  A channel
 * slice of a larger tensor is a view with a shifted data pointer and the
 * larger tensor's c_stride (and a slot pointer shifted by c0 / 16). */
typedef struct AexrtHipTensorView {
    void* data;
    int64_t n_stride;
    int32_t c_stride;
    uint32_t amax_stripes;
    uint32_t* amax_slots;
    uint64_t amax_stripe_stride;
} AexrtHipTensorView;

/* Conv flags (aexrt_hip_conv2d). */
#define AEXRT_HIP_CONV_SILU 1u     /* SiLU after bias (CONV_SILU commands)        */
#define AEXRT_HIP_CONV_RESIDUAL 2u /* + residual view after the activation        */
#define AEXRT_HIP_CONV_OUT_F32 4u  /* fp32 output view instead of fp16             */
#define AEXRT_HIP_CONV_IN_NCHW_F32 8u /* x->data is a dense fp32 NCHW tensor (network
                                       * input of the stem conv): c = x->n_stride / (H*W)
                                       * <= 4 channels, read as in_channels = 8 (weights
                                       * packed for 8, zero past c); fp16 3x3 pad-1 SiLU
                                       * convs with fp16 output only */
#define AEXRT_HIP_CONV_INT8_PG16 16u  /* int8 with per-16-input-channel activation scales
                                       * (plan flag 16, native/aexrt_d3d12_runtime.cpp:
                                       * 4770-4923): slot g of x->amax_slots is group g's
                                       * amax (the reference's amax[1 + g]); no acc_out */
#define AEXRT_HIP_CONV_INT8_DYNAMIC 32u /* int8 with the scale computed in the kernel per output
                                         * position and 4-channel input group (the reference's
                                         * fallback int8 conv, native/aexrt_d3d12_runtime.cpp:
                                         * 2952-3115, dispatched for inputs of fewer than 4096
                                         * elements, RT:21478-21479); x->amax_slots is not read;
                                         * no acc_out, not with PG16 */

/* Weight source layouts accepted by aexrt_hip_pack_conv_weight: the
 * reference's packed layouts (src/aexrt/engine.py:59-71) plus raw constants. */
#define AEXRT_HIP_SRC_RAW_F32 0u          /* [oc][ic][kh][kw] fp32 constant              */
#define AEXRT_HIP_SRC_RAW_F16 1u          /* [oc][ic][kh][kw] fp16 constant (precision 2) */
#define AEXRT_HIP_SRC_LAYOUT_OC4_F16 2u   /* layout 2: [oc/4][ic][9][4] fp16              */
#define AEXRT_HIP_SRC_LAYOUT_WINO_F16 3u  /* layout 3: [oc][ic][4][4] fp16 U = G g G^T    */
#define AEXRT_HIP_SRC_LAYOUT_OC8_F16 4u   /* layout 4: [oc/8][ic][8] fp16 (1x1)           */
#define AEXRT_HIP_SRC_LAYOUT_WINO_F32 5u  /* layout 5: [oc][ic][4][4] fp32                */
#define AEXRT_HIP_SRC_LAYOUT_INT8 8u      /* layout 8: int8 [oc][ic][kk] + oc fp32 scales */

/* ---------------------------------------------------------------------- */
/* Library / errors                                                        */
/* ---------------------------------------------------------------------- */

/* Version of this ABI (bumped on incompatible changes). */
uint32_t aexrt_hip_abi_version(void);
/* Last error of the calling thread (op-level calls and model creation);
 * same role as the global fallback of aexrt_yolo_get_last_error
 * (native/aexrt_d3d12_runtime.cpp:27798-27816). */
const char* aexrt_hip_get_last_error(void);

/* ---------------------------------------------------------------------- */
/* Op-level entry points (device pointers; stream = hipStream_t or NULL)   */
/* ---------------------------------------------------------------------- */

/* a1, producer-side form: atomically folds max|x| of every 16-channel group
 * of an NHWC fp16 view into x->amax_slots (which the caller clears first).
 * Replaces the zero + amax dispatches (native/aexrt_d3d12_runtime.cpp:
 * 3193-3259, recorded at 21622-21644). */
int aexrt_hip_amax_slots(const AexrtHipTensorView* x, uint32_t batch, uint32_t height,
                         uint32_t width, uint32_t channels, void* stream);

/* a1, reference form: the reference's amax buffer over an NCHW tensor
 * (fp16 when is_f16, else fp32).  out[0] = per-tensor max, out[1+g] = max
 * over memory strip g of 16*N*H*W elements; out has C/16+1 words and is
 * cleared by this call (native/aexrt_d3d12_runtime.cpp:3219-3259). */
int aexrt_hip_amax_nchw(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels,
                        uint32_t plane, uint32_t* out, void* stream);

/* a2, layout-free form: int8 NHWC (dense, [N*H*W][C]) = round_half_even(
 * x * 127/amax) with amax = max of the view's amax slots
 * (native/aexrt_d3d12_runtime.cpp:3337-3344). */
int aexrt_hip_quantize(const AexrtHipTensorView* x, uint32_t batch, uint32_t height,
                       uint32_t width, uint32_t channels, int8_t* q, void* stream);

/* a2, reference form: NC/4HW4 uint32 pack of an NCHW tensor with amax[0]
 * (per_group = 0) or amax[1 + icg/4] (per_group = 1)
 * (native/aexrt_d3d12_runtime.cpp:3314-3346). */
int aexrt_hip_quant_pack_nchw(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels,
                              uint32_t plane, const uint32_t* amax, uint32_t per_group,
                              uint32_t* packed, void* stream);

/* a1 strips over an NHWC fp16 view, for pg16 scales: max|x| of image n and
 * channel group g is folded into out[(n * C/16 + g) / N], which is the
 * reference's amax[1 + s] of memory strip s of 16*N*H*W elements of the same
 * tensor in NCHW layout (native/aexrt_d3d12_runtime.cpp:3219-3259).  out
 * (C/16 words) is cleared by this call; x->amax_slots is not used. */
int aexrt_hip_amax_strips_nhwc(const AexrtHipTensorView* x, uint32_t batch, uint32_t height,
                               uint32_t width, uint32_t channels, uint32_t* out, void* stream);

/* a3: the reference's fused pg16 amax + pack of an NCHW tensor (fp16 when
 * is_f16, else fp32), native/aexrt_d3d12_runtime.cpp:4083-4149: amax[1 + g]
 * = max|x| over channels 16g..16g+15 of image 0 (used for every image, as
 * in the reference), packed = NC/4HW4 int8 words of every image quantized
 * with 127/amax[1 + g].  amax[0] is not written.  C % 16 == 0. */
int aexrt_hip_quant_fused_pg16(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels,
                               uint32_t plane, uint32_t* packed, uint32_t* amax, void* stream);

/* a4 (load side): size and host-side repack of a conv weight into the
 * layout the kernel of `algorithm` consumes.  algorithm is the reference's
 * AexrtTileFlowConvAlgorithm id (native/aexrt_d3d12_runtime.cpp:8881-8940):
 * 51/52/53 -> int8 MFMA ([OCp][Kp] int8, K = (ky,kx,c)), 40/46 -> Winograd
 * ([16][OCp][Cp] fp16), anything else -> fp16 MFMA ([OCp][Kp] fp16).
 * For int8 the oc scales are written to scale_out (oc floats).  Mirrors the
 * reference's upload repack (native/aexrt_d3d12_runtime.cpp:21744-21773). */
int aexrt_hip_conv_weight_bytes(const AexrtConv2DDesc* desc, uint32_t algorithm,
                                uint64_t* out_nbytes);
int aexrt_hip_pack_conv_weight(const AexrtConv2DDesc* desc, uint32_t algorithm,
                               uint32_t src_layout, const void* src, uint64_t src_nbytes,
                               void* dst, uint64_t dst_nbytes, float* scale_out);

/* a5/a7/a12/a13: one convolution on device views.  x, residual and y are
 * NHWC views (fp16; y fp32 with AEXRT_HIP_CONV_OUT_F32).  For int8
 * algorithms the quantization scale comes from x->amax_slots (C/16 slots)
 * and w_scale holds the oc weight scales; acc_out (optional, int32
 * [N*OH*OW][OC]) receives the exact accumulators.  When y->amax_slots is
 * set the epilogue folds max|y| into it.  Replaces record_replay_conv's
 * dispatch (native/aexrt_d3d12_runtime.cpp:23280-24318). */
int aexrt_hip_conv2d(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                     const AexrtHipTensorView* x, const void* weight, const float* w_scale,
                     const float* bias, const AexrtHipTensorView* residual,
                     const AexrtHipTensorView* y, int32_t* acc_out, void* stream);

/* An int8 1x1 conv (algorithm 51/52/53, per-tensor, the arguments of
 * aexrt_hip_conv2d without residual and accumulators) that also writes the
 * nearest 2x upsample of its fp16 output into y_up (2 OH x 2 OW positions per
 * image, OC channels: e.g. the channel slice of a concat that a resize of y
 * used to fill) and folds its amax into y_up's slots.  Replaces the
 * reference's RESIZE command on a conv output (src/aexrt/yolo.py:830-834;
 * the nearest resize shader native/aexrt_d3d12_runtime.cpp:14851-14872, which
 * reads y again and writes y_up) with stores in the conv's own launch.
 * Runs on the streaming 1x1 kernel (a tile forced with
 * aexrt_hip_set_conv1x1_stream, else the first that fits); 0 with a
 * diagnostic when none fits (fp32 output, views). */
int aexrt_hip_conv2d_upsample_copy(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                   const AexrtHipTensorView* x, const void* weight, const float* w_scale,
                                   const float* bias, const AexrtHipTensorView* y, const AexrtHipTensorView* y_up,
                                   void* stream);

/* An int8 1x1 conv (algorithm 51/52/53, per-tensor, the arguments of
 * aexrt_hip_conv2d without residual) whose input channels [up_c0, up_c0 +
 * up_channels) are the nearest 2x upsample of x_up (a map of H/2 x W/2
 * positions with its own amax slots), read from x_up directly: x's memory for
 * those channels is not read, and the per-tensor amax is the max over x's
 * other slots and x_up's.  Replaces the reference's RESIZE into a concat
 * slice followed by the concat's 1x1 conv (src/aexrt/yolo.py:830-834, the
 * CONCAT_CONV1X1 pattern yolo.py:473-488; shaders
 * native/aexrt_d3d12_runtime.cpp:14851-14872 and 4614-4762) with the conv
 * alone, the upsample never stored.  x and x_up must lie within one 4 GB
 * span (one arena, as a model's values do).  acc_out: optional int32 sums.
 * Runs on
 * the streaming 1x1 kernel (a forced tile, else the first that fits); 0 with
 * a diagnostic when none fits. */
int aexrt_hip_conv2d_upsampled_input(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                     const AexrtHipTensorView* x, const AexrtHipTensorView* x_up, uint32_t up_c0,
                                     uint32_t up_channels, const void* weight, const float* w_scale,
                                     const float* bias, const AexrtHipTensorView* y, int32_t* acc_out, void* stream);

/* The kernel and tile candidates the model loader measures for one conv
 * (no reference counterpart; the tile-level analogue of the algorithm
 * candidates of aexrt_yolo_conv_plan_info, native/aexrt.h:435-445, and of
 * replay_conv_algorithm's candidate list, RT:9510-9576).  x, residual and y
 * give the views' strides (pointers only need to be 16-byte aligned and
 * non-null; nothing is read).  For each candidate i < cap, names + i *
 * name_len receives the kernel instance and tile its launcher would run
 * ("" when the launcher rejects it).  Returns the candidate count, which
 * can exceed cap; no kernel runs and no HIP call is made.  Winograd, pg16
 * and dynamic int8 convs have no tile choice: 0 with a diagnostic. */
uint32_t aexrt_hip_conv_candidates(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                   const AexrtHipTensorView* x, const AexrtHipTensorView* residual,
                                   const AexrtHipTensorView* y, char* names, uint32_t name_len,
                                   uint32_t cap);

/* C2f bottleneck superblock (the reference's fusion kind 1,
 * src/aexrt/engine.py:75-76, shader native/aexrt_d3d12_runtime.cpp:
 * 12205-12563, there in fp32): conv a (3x3 s1 p1 SiLU, C -> C) and conv b
 * (the same, plus x as residual with AEXRT_HIP_CONV_RESIDUAL) in one
 * launch, a's output kept on chip.  desc is conv a's (and b's) descriptor:
 * C = in = out channels, a multiple of 32 up to 128.  algorithm 52: W8A8
 * (x->amax_slots give x's per-tensor scale; the intermediate is quantized
 * with its own per-tensor amax over the whole batch, exchanged between the
 * workgroups through a grid barrier, exactly as two int8 convs would), or
 * an fp16 id.  Weights packed for `algorithm` (aexrt_hip_pack_conv_weight),
 * w_scale_* for int8.  y: fp16 NHWC view, its amax slots folded when set.
 * band_rows: output rows per workgroup (0: chosen).  Optional: t_out (fp16
 * dense NHWC copy of the intermediate), acc_a / acc_b (int32 [N*H*W][C]
 * sums of the two convs, int8).  Returns 0 with a diagnostic when the
 * shape, the band or (int8) the whole grid at once does not fit the GPU.
 * Asynchronous on `stream`; the int8 form uses a per-device sync area
 * (overlapping int8 calls on one device race). */
int aexrt_hip_conv_pair(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                        const AexrtHipTensorView* x, const void* weight_a, const float* w_scale_a,
                        const float* bias_a, const void* weight_b, const float* w_scale_b,
                        const float* bias_b, const AexrtHipTensorView* y, uint32_t band_rows,
                        void* t_out, int32_t* acc_a, int32_t* acc_b, void* stream);
/* Synchronizes the device and returns the barrier-timeout word of the int8
 * pair entry's sync area on the current device (0: every grid barrier
 * completed; the wait is bounded and sets this word instead of hanging). */
uint32_t aexrt_hip_conv_pair_barrier_timeouts(void);

/* a15 on the GPU: fp32 direct convolution of dense NCHW tensors, the
 * reference's aexrt_d3d12_conv2d_float32 / aexrt_d3d12_conv2d_silu_float32
 * (native/aexrt.h:175-189; shader native/aexrt_d3d12_runtime.cpp:1554-1622)
 * with the arithmetic of its CPU path cpu_conv2d (RT:20552-20580): acc =
 * bias[oc], then += x*w over (input channel of the group, ky, kx), taps
 * outside the input skipped, each multiply and add rounded on its own;
 * flags AEXRT_HIP_CONV_SILU: acc / (1 + exp(-acc)).  weight [OC][C/groups]
 * [KH][KW] fp32; x [N][C][H][W]; y [N][OC][OH][OW]; any stride, padding,
 * dilation and groups. */
int aexrt_hip_conv2d_f32(const AexrtConv2DDesc* desc, uint32_t flags, const float* x, const float* weight,
                         const float* bias, float* y, void* stream);

/* a14 for int8 commands: the reference's whole int8 conv command (the int8
 * block of record_replay_conv, native/aexrt_d3d12_runtime.cpp:23935-24318)
 * on a plain fp16 NHWC input view (x->amax_slots is ignored):
 *   - an input of fewer than 4096 elements (RT:21478-21479) runs the dynamic
 *     kernel (per position and 4-channel group scales, RT:2952-3115);
 *   - with AEXRT_HIP_CONV_INT8_PG16 the reference's strip amax of the input
 *     (RT:3219-3259) then the pg16 conv (RT:4770-4923);
 *   - otherwise the per-tensor amax of the input, then the prequantized conv
 *     (RT:3314-3346, 4614-4762) quantizing on load.
 * algorithm 51/52/53; flags SILU / RESIDUAL / OUT_F32 / INT8_PG16; in_channels
 * % 16 == 0.  The amax words live in a scratch buffer the library allocates
 * on the current device at first use (16 x C/16 uint32, grown when a conv
 * needs more) and keeps until the process ends; every call clears what it
 * uses first.  Calls that overlap on one device share that scratch and race. */
int aexrt_hip_conv2d_int8(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView* x,
                          const void* weight, const float* w_scale, const float* bias,
                          const AexrtHipTensorView* residual, const AexrtHipTensorView* y, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): aexrt_hip_conv2d_int8 with its amax scratch in a static
 * device array of 16 KiB (16 x 256 uint32) that each device holds until the
 * process ends, instead of library-allocated memory; calls no allocating
 * routine.  Same arguments, kernels and results as aexrt_hip_conv2d_int8;
 * in_channels <= 4096, larger convs are refused with a diagnostic.  Every
 * call on a device shares that device's array (cleared before use): calls
 * that overlap on one device race. */
int aexrt_hip_conv2d_int8_noalloc(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                  const AexrtHipTensorView* x, const void* weight, const float* w_scale,
                                  const float* bias, const AexrtHipTensorView* residual, const AexrtHipTensorView* y,
                                  void* stream);

/* a6, reference form: the pg16 int8 conv on the reference's own operands,
 * native/aexrt_d3d12_runtime.cpp:4770-4923 (dispatch 24152-24258): packed =
 * NC/4HW4 int8 words (aexrt_hip_quant_pack_nchw with per_group = 1, or
 * aexrt_hip_quant_fused_pg16), amax = that buffer (amax[1 + g] scales group
 * g), weight packed by aexrt_hip_pack_conv_weight for algorithm 51/52/53,
 * w_scale/bias per output channel.  y = dense NCHW, fp16, or fp32 with
 * AEXRT_HIP_CONV_OUT_F32; flags also AEXRT_HIP_CONV_SILU.  in_channels % 16
 * == 0 (<= 4096). */
int aexrt_hip_conv2d_int8_pg16(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                               const uint32_t* packed, const uint32_t* amax, const void* weight,
                               const float* w_scale, const float* bias, void* y, void* stream);

/* YOLO postprocess on one output0 image in device memory, the reference's
 * dispatch_yolo_decode_nms_float32 (native/aexrt_d3d12_runtime.cpp:
 * 15300-15356, 15637-15735): layout 2 = channels last ([anchors][channels]),
 * otherwise channels first.  A candidate is an anchor whose best class score
 * (times objectness) is not below conf_threshold, at most max_candidates of
 * them in anchor order; one is dropped when a candidate of its class with a
 * higher score (equal: earlier) overlaps it with IoU > iou_threshold;
 * detections = the kept ones by score, at most max_detections, written as
 * [count][6] floats with *count (device memory).  max_candidates <= 2048. */
int aexrt_hip_yolo_decode_nms_topk(const float* output, uint32_t layout, uint32_t anchors, uint32_t channels,
                                   uint32_t classes, uint32_t has_objectness, float conf_threshold,
                                   float iou_threshold, uint32_t max_candidates, uint32_t max_detections,
                                   float* detections, uint32_t* count, void* stream);

/* YOLO postprocess on the raw Detect head of one image (the post-conv part
 * of the reference's fused head decode, native/aexrt_d3d12_runtime.cpp:
 * 15465-15636, then NMS and top-k as above): head = [64 + classes][anchors]
 * fp32 (layout 2: [anchors][64 + classes]), channels 0..63 the 4 x 16 DFL
 * bin logits (side-major), then the class logits; anchors level by level,
 * level l a level_hw[2l] x level_hw[2l+1] grid with stride level_strides[l].
 * score = sigmoid(logit); side distance = softmax expectation of its 16
 * bins; box = ((gx + 0.5 - l) s, (gy + 0.5 - t) s, (gx + 0.5 + r) s,
 * (gy + 0.5 + b) s).  exp is computed by Cody-Waite reduction and a
 * degree-7 Taylor polynomial (the reference's comes from its shader
 * compiler).  level_hw and level_strides are host arrays. */
int aexrt_hip_yolo_dfl_decode_nms_topk(const float* head, uint32_t layout, uint32_t num_levels,
                                       const uint32_t* level_hw, const float* level_strides, uint32_t classes,
                                       float conf_threshold, float iou_threshold, uint32_t max_candidates,
                                       uint32_t max_detections, float* detections, uint32_t* count, void* stream);

/* a10: int8 eligibility of a conv for kernel family kernel_elems (1 or 9),
 * native/aexrt_d3d12_runtime.cpp:9399-9422, plus this backend's own
 * requirement in_channels % 16 == 0 (amax is kept per 16 channels). */
int aexrt_hip_can_use_conv_int8(const AexrtConv2DDesc* desc, uint32_t kernel_elems);

/* Tuning/test hook with no counterpart in the reference: forces the
 * implicit-GEMM conv kernel onto one per-wave tile (jn 16-channel x pw
 * 16-position subtiles; ksw = the 4 waves of a block split k, pw must be 1)
 * for every following launch in the process; (0, 0, 0) restores the
 * automatic choice.  Returns 0 for a tile without a kernel instance. */
int aexrt_hip_set_conv_tile(int32_t jn, int32_t pw, int32_t ksw);
/* Tuning/test hook, no reference counterpart: 3x3 pad-1 convs with C % 16 == 0
 * run on the halo-tile kernel (input window staged and quantized once in LDS).
 * mode 0 = automatic tile, 1 = never (implicit GEMM for every conv), 2 = force
 * the tile with 4 waves per block, 3 = with 8 waves (pw 1 or 2): jn 16-channel
 * subtiles (1/2/4), pw 16-position subtiles per wave (1/2/4), tr x tc output
 * positions (tr * tc <= 16 * waves * pw), cc input channels per LDS chunk
 * (C % cc == 0; cc % 16 == 0 for int8, % 8 for fp16); a 3x3 conv that the
 * forced tile does not fit (LDS, channel chunk) then fails.  jn 5 (80
 * channels) exists with 8 waves.  mode 4 = force the wide-tile fp16 kernel on
 * fp16 convs (every output channel, 49..80, in each wave; jn 4 or 5, pw 2 or
 * 4, tr * tc <= 64 * pw, cc channels per chunk with weights streamed).
 * mode 5 = force the 32x32-MFMA kernel on 3x3 convs (int8 and fp16, C % 16 ==
 * 0) with 4 waves per block: jn 32-channel subtiles per block (1..4; 1..2
 * with pw 4), pw 32-position subtiles per wave (1/2/4), tr x tc output
 * positions (tr * tc <= 128 * pw), cc input channels per chunk (C % cc == 0,
 * cc % 16 == 0; the weights of all chunks stay in LDS); mode 6 = the same
 * with 8 waves per block (pw 1 with jn 1..3, pw 2 with jn 1..2; tr * tc <=
 * 256 * pw); mode 7 = 8 waves in two groups of 4, each group with its own
 * input windows and barrier and its own tiles of the block's run (pw 1 with
 * jn 1..3, pw 2 with jn 1..2; tr * tc <= 128 * pw).  Any other mode
 * switches modes 5, 6 and 7 off.
 * Returns 0 for a bad request. */
int aexrt_hip_set_conv3x3_halo(int32_t mode, int32_t jn, int32_t pw, int32_t tr, int32_t tc, int32_t cc);

/* fp16 3x3 SiLU conv (algorithm 5 weights) with a 1x1 conv of its output fused
 * into the epilogue: y2 = conv1x1(fp16(silu(conv3x3(x) + bias)), weight2) +
 * bias2 (SiLU when flags2 has it, fp32 y2 with OUT_F32); the 3x3 output is
 * never stored.  The
 * YOLOv8 head's last two convs of each branch (the reference fuses its head
 * into one replay group, fusion kinds 4/5 of src/aexrt/engine.py:78-79).
 * Runs on the 32x32-MFMA kernel with a tile covering every 3x3 output channel
 * (<= 96): the one forced by aexrt_hip_set_conv3x3_halo mode 5/6, else the
 * first that fits.  flags = SILU; y2 gets amax slots when its view has them.
 * Returns 0 and sets the error otherwise. */
int aexrt_hip_conv2d_fused_1x1(const AexrtConv2DDesc* desc, uint32_t flags, const AexrtHipTensorView* x,
                               const void* weight, const float* bias, const AexrtConv2DDesc* desc2, uint32_t flags2,
                               const void* weight2, const float* bias2, const AexrtHipTensorView* y2, void* stream);

/* A detect-head branch in one launch: y = conv_c(t2), t2 = fp16(silu(conv_b(t1)
 * + bias_b)), t1 = fp16(silu(conv_a(x) + bias_a)); a and b fp16 3x3 stride-1
 * pad-1 convs (algorithm 5 weights), b over a's output, c a 1x1 conv over b's
 * output (flags_c: SILU, OUT_F32; y without amax slots); every conv at most 96
 * output channels, the 3x3 inputs in 16-channel steps.  t1 and t2 stay in the
 * kernel's LDS (one tile of tile_rows x tile_cols outputs per block plus the
 * border conv b needs, recomputed by neighbouring tiles; 0 x 0: chosen) and
 * are never stored.  The reference runs these three convs of each head
 * branch inside its fused head replay group (fusion kinds 4/5,
 * src/aexrt/engine.py:78-79).  Returns 0 and sets the error otherwise. */
int aexrt_hip_conv_chain3(const AexrtConv2DDesc* desc_a, const void* weight_a, const float* bias_a,
                          const AexrtConv2DDesc* desc_b, const void* weight_b, const float* bias_b,
                          const AexrtConv2DDesc* desc_c, uint32_t flags_c, const void* weight_c, const float* bias_c,
                          const AexrtHipTensorView* x, const AexrtHipTensorView* y, uint32_t tile_rows,
                          uint32_t tile_cols, void* stream);

/* Tuning/test hook, no reference counterpart: mode 1 runs every int8 1x1
 * stride-1 conv launched without a measured kernel choice on the streaming
 * 1x1 kernel (weights resident in LDS, each tile's input loaded at once and
 * quantized once into an int8 LDS tile) with jq 16-channel subtiles per block
 * (1/2/4/8) and pq 16-position subtiles per wave (1, or 2 with jq <= 4); a
 * conv that tile does not fit (LDS, views not evenly strided, residual) then
 * fails.  mode 2: the same on a grid of one tile per block instead of a
 * persistent grid.  mode 0 switches it off.  Returns 0 for a tile without an
 * instance. */
int aexrt_hip_set_conv1x1_stream(int32_t mode, int32_t jq, int32_t pq);

/* Kernel of the network's first conv (3x3 pad 1, stride 1/2, the fp32 NCHW
 * input with at most 3 channels read directly, SiLU, fp16 output; a kernel
 * choice of the reference's replay_conv_algorithm, RT:9424-9500): mode 0
 * automatic (a band kernel of whole output rows when the conv fits it),
 * 1 never (the halo-tile kernel), 2 forced band of tr output rows on a grid
 * of resident blocks, 3 the same with one band per block (a conv the band
 * does not fit then fails).  Returns 0 for a bad request. */
int aexrt_hip_set_conv_stem(int32_t mode, int32_t tr);

/* Glue ops of the replay stream on NHWC fp16 views. */
int aexrt_hip_fill_u32(uint32_t* dst, uint64_t count, uint32_t value, void* stream);
int aexrt_hip_nchw_f32_to_nhwc(const float* x, uint32_t batch, uint32_t channels, uint32_t plane,
                               const AexrtHipTensorView* y, void* stream);
int aexrt_hip_nhwc_to_nchw_f32(const AexrtHipTensorView* x, uint32_t is_f16, uint32_t batch,
                               uint32_t channels, uint32_t plane, float* y, void* stream);
int aexrt_hip_copy(const AexrtHipTensorView* src, const AexrtHipTensorView* dst, uint32_t batch,
                   uint32_t plane, uint32_t channels, void* stream);
int aexrt_hip_maxpool(const AexrtHipTensorView* x, const AexrtHipTensorView* y, uint32_t batch,
                      uint32_t channels, uint32_t in_h, uint32_t in_w, uint32_t out_h,
                      uint32_t out_w, uint32_t kernel, uint32_t stride, uint32_t pad, void* stream);
/* SPPF's three chained MAXPOOL commands (5x5, stride 1, pad 2; RT's MAXPOOL
 * replay, invoked three times in a row) in one pass: y1 = pool(x), y2 =
 * pool(y1), y3 = pool(y2), with their amax slots.  No reference counterpart as
 * one call (the runtime folds the three commands into it); y1..y3 share one
 * geometry (slices of one concat tensor). */
int aexrt_hip_sppf_maxpool(const AexrtHipTensorView* x, const AexrtHipTensorView* y1,
                           const AexrtHipTensorView* y2, const AexrtHipTensorView* y3, uint32_t batch,
                           uint32_t channels, uint32_t h, uint32_t w, void* stream);
int aexrt_hip_resize_nearest(const AexrtHipTensorView* x, const AexrtHipTensorView* y,
                             uint32_t batch, uint32_t channels, uint32_t in_h, uint32_t in_w,
                             uint32_t out_h, uint32_t out_w, void* stream);
int aexrt_hip_add(const AexrtHipTensorView* a, const AexrtHipTensorView* b,
                  const AexrtHipTensorView* y, uint32_t batch, uint32_t plane, uint32_t channels,
                  void* stream);

/* ---------------------------------------------------------------------- */
/* Model-level API (native/aexrt.h YOLO entry points)                      */
/* ---------------------------------------------------------------------- */

typedef struct AexrtDevice AexrtDevice;
typedef struct AexrtYoloModel AexrtYoloModel;

/* Replaces AexrtD3D12Capabilities (native/aexrt.h:29-37) for a HIP device. */
typedef struct AexrtHipCapabilities {
    uint32_t struct_size;
    uint32_t device_index;
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint32_t lds_bytes_per_block;
    uint32_t int8_mfma;     /* 1 when v_mfma_i32_16x16x64_i8 is available (gfx950) */
    uint32_t fp16_mfma;
    uint32_t reserved;
    uint64_t global_mem_bytes;
    char arch_name[64];
} AexrtHipCapabilities;

/* native/aexrt.h:43-51 */
typedef struct AexrtYoloRunTiming {
    uint32_t struct_size;
    uint32_t valid;
    double memcpy_ms;   /* host input copy into the model's device input buffer */
    double submit_ms;   /* graph launch (or kernel launches) */
    double fence_ms;    /* stream synchronisation */
    double readback_ms; /* result readback */
    uint64_t reserved[4];
} AexrtYoloRunTiming;

/* native/aexrt.h:435-445 */
typedef struct AexrtConvPlanInfo {
    uint32_t struct_size;
    uint32_t command_index;
    uint32_t kind_is_silu;
    AexrtConv2DDesc desc;
    uint32_t current_algorithm;
    uint32_t candidate_count;
    uint32_t candidates[32];
    uint32_t in_fusion_group;
    uint32_t planned_algorithm;
} AexrtConvPlanInfo;

/* Device handle (replaces aexrt_d3d12_create_device / destroy_device /
 * get_capabilities, native/aexrt.h:129-140). */
AexrtDevice* aexrt_hip_create_device(uint32_t device_index);
void aexrt_hip_destroy_device(AexrtDevice* device);
int aexrt_hip_get_capabilities(AexrtDevice* device, AexrtHipCapabilities* caps);

/* native/aexrt.h:29-37, the struct the reference's wrapper passes. */
typedef struct AexrtD3D12Capabilities {
    uint32_t struct_size;
    uint32_t highest_shader_model; /* 0: no D3D shader model (HIP code objects)   */
    uint32_t native_fp16_supported; /* 1                                          */
    uint32_t wave_mma_tier;         /* 1 with matrix cores (gfx950 MFMA), else 0  */
    uint32_t dxc_available;         /* 0                                          */
    uint32_t reserved[3];
} AexrtD3D12Capabilities;

/* The reference's device entry points under their own names
 * (native/aexrt.h:129-140; bound by src/aexrt/cpp_runtime.py:543-548), so
 * its ctypes wrapper loads this library with only the path changed:
 * probe = 1 when a HIP device exists; create/destroy = the aexrt_hip_ ones
 * (adapter_index = HIP device index). */
int aexrt_d3d12_probe(void);
AexrtDevice* aexrt_d3d12_create_device(uint32_t adapter_index);
void aexrt_d3d12_destroy_device(AexrtDevice* device);
int aexrt_d3d12_get_capabilities(AexrtDevice* device, AexrtD3D12Capabilities* capabilities);

/* native/aexrt.h:271-281: building from a package directory or an ONNX file
 * is the compiler's job here (aexrt_amd.engine writes the .aexrt engine):
 * both return NULL with a diagnostic; load engines with
 * aexrt_yolo_load_engine. */
AexrtYoloModel* aexrt_yolo_compile_from_package(AexrtDevice* device, const char* package_path);
AexrtYoloModel* aexrt_yolo_compile_from_onnx(AexrtDevice* device, const char* onnx_path);

/* native/aexrt.h:275: load a .aexrt engine (sections 1-9 required, 10-11
 * accepted; the reference loader's record rules, RT:17560-18593, CRC per
 * section; fail closed).  The _memory variant takes the engine bytes
 * directly. */
AexrtYoloModel* aexrt_yolo_load_engine(AexrtDevice* device, const char* engine_path);
/* Parses and validates engine bytes without a device, including the shape
 * checks of the load (1 = loadable). */
int aexrt_hip_validate_engine(const void* data, uint64_t nbytes);
AexrtYoloModel* aexrt_yolo_load_engine_memory(AexrtDevice* device, const void* data, uint64_t nbytes);

/* native/aexrt.h:283-330 model queries. */
uint64_t aexrt_yolo_input_element_count(AexrtYoloModel* model);
uint64_t aexrt_yolo_output_element_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_class_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_anchor_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_channel_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_output_layout(AexrtYoloModel* model);
uint32_t aexrt_yolo_has_objectness(AexrtYoloModel* model);
uint32_t aexrt_yolo_graph_node_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_graph_value_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_constant_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_prepared_command_count(AexrtYoloModel* model);  /* engine-file commands */
int aexrt_yolo_is_executable(AexrtYoloModel* model);

/* native/aexrt.h:301: 2 (AEXRT_YOLO_PACKAGE_NATIVE_D3D12_GRAPH) for an
 * engine, the reference's value for .aexrt models (RT:17627). */
uint32_t aexrt_yolo_package_mode(AexrtYoloModel* model);
/* native/aexrt.h:313-385, the prepared-plan counters (RT:29204-29285,
 * 22913-23110), for what this runtime does with the engine's commands:
 *   supported = every command (the loader refuses engines it cannot run),
 *   unsupported = 0;
 *   skipped = engine commands with no launch of their own (views, aliases,
 *   concats placed in place, residual adds in a conv epilogue, the 2nd/3rd
 *   SPPF pools, the second conv of a paired launch);
 *   late_concat_conv1x1 = concats placed in place whose output a 1x1 conv
 *   reads whole; paired_conv3x3 = pairs of 3x3 convs of one input computed
 *   by one launch; c2f_tail_residual = residual adds done in a conv
 *   epilogue; concat_residual_conv1x1, c2f_bottleneck_superblock and the
 *   head fusions = 0 (D3D12 fusions this backend does not form);
 *   tileflow_* = convs by the kernel family that runs them: conv1x1 = 1x1
 *   convs; 3x3_spatial = 3x3 convs on a spatial tile kernel (halo window,
 *   wide, band); 3x3_pack4 = 3x3 convs on the dynamic int8 dot4 kernel;
 *   3x3_pack8 = 0; 3x3_implicit_gemm = 3x3 convs on the implicit-GEMM,
 *   pg16 or Winograd kernels, with 40x40 / 20x20 / 10x10 and exact-shape
 *   sub-counts; native_fp16 = convs on fp16 MFMA kernels. */
uint32_t aexrt_yolo_supported_prepared_command_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_unsupported_prepared_command_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_prepared_skipped_command_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_late_concat_conv1x1_fusion_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_concat_residual_conv1x1_fusion_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_paired_conv3x3_fusion_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_c2f_bottleneck_superblock_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_c2f_tail_residual_fusion_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_head_fusion_enabled(AexrtYoloModel* model);
uint32_t aexrt_yolo_head_final_conv_fusion_enabled(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_conv1x1_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_spatial_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_pack4_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_pack8_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_40x40_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_20x20_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_10x10_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_exact_40x40_64x64_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_exact_20x20_64x64_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_exact_10x10_128x128_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_exact_20x20_128x64_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_3x3_exact_10x10_256x64_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_tileflow_native_fp16_count(AexrtYoloModel* model);

/* native/aexrt.h:412-421: runs are synchronous (no frame in flight), so a
 * flush returns 1 with 0 detections, as the reference does with one
 * pipeline frame; 0 on a null argument or max_detections == 0. */
int aexrt_yolo_flush_pipeline(AexrtYoloModel* model, AexrtYoloDetection* detections, uint32_t max_detections,
                              uint32_t* out_detection_count);

/* native/aexrt.h:469-484: no shader or pipeline objects are compiled at
 * load, so the exported cache is the valid empty one (16 bytes: version 1,
 * 0 shader and 0 PSO records, flags 1, as RT:31062-31101 writes it with no
 * entries) and the hit counts are 0. */
uint64_t aexrt_yolo_pipeline_cache_size(AexrtYoloModel* model);
int aexrt_yolo_export_pipeline_cache(AexrtYoloModel* model, void* output, uint64_t output_nbytes);
uint32_t aexrt_yolo_dxil_cache_hit_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_shader_cache_hit_count(AexrtYoloModel* model);
uint32_t aexrt_yolo_pso_cache_hit_count(AexrtYoloModel* model);

/* native/aexrt.h:391-398: one inference from a host fp32 CHW input.  The
 * network and the YOLO postprocess of output0 (decode + confidence filter,
 * class-wise NMS, top-k; native/aexrt_d3d12_runtime.cpp:27104-27219) run on
 * the device; *out_detection_count = min(detections found, max_detections,
 * the engine's max_detections), best score first.  Engines whose output is
 * not a YOLO head (manifest channels/anchors/classes do not match output0)
 * report 0 detections; the raw output is available through
 * aexrt_yolo_debug_output. */
int aexrt_yolo_run(AexrtDevice* device, AexrtYoloModel* model, const float* input,
                   uint64_t input_element_count, AexrtYoloDetection* detections,
                   uint32_t max_detections, uint32_t* out_detection_count);

/* Device-resident run: when input is non-NULL it is a device fp32 NCHW
 * tensor copied into the model's input buffer first; the network then runs
 * on `stream` (NULL = the model's own stream).  No host synchronisation. */
int aexrt_yolo_run_device(AexrtYoloModel* model, const float* input, void* stream, void* reserved);
/* Device-side postprocess of the last run's output0 on `stream` (NULL = the
 * model's stream), without host synchronisation: *detections_device gets the
 * model's [max_detections][6] float buffer (x1, y1, x2, y2, score, class) and
 * *count_device its uint32 detection count.  No counterpart in the reference
 * (whose run always reads back); for callers that keep results in HBM. */
int aexrt_yolo_postprocess_device(AexrtYoloModel* model, void* stream, float** detections_device,
                                  uint32_t** count_device);
/* Device pointers of the model's input (fp32 NCHW) and output buffers. */
void* aexrt_yolo_input_device_ptr(AexrtYoloModel* model);
/* native/aexrt.h:465 zero-copy host input (pinned). */
void* aexrt_yolo_input_ptr(AexrtYoloModel* model, uint64_t* out_elements);

/* native/aexrt.h:401-403: read back a value / the output as fp32 in the
 * logical NCHW (or [N, C, A]) order. */
int aexrt_yolo_debug_output(AexrtYoloModel* model, float* out, uint64_t elements);
int aexrt_yolo_debug_value(AexrtYoloModel* model, uint32_t value_id, float* out, uint64_t elements);
/* native/aexrt.h:403 reads a D3D12 arena page; values here live in one NHWC
 * arena read through debug_value: returns 0 with a diagnostic. */
int aexrt_yolo_debug_page(AexrtYoloModel* model, uint32_t page_id, float* out, uint64_t elements);
/* Debug tap of a per-tensor int8 conv of the loaded model (no reference
 * counterpart; it exposes the reference's bit-exact quantities,
 * native/aexrt_d3d12_runtime.cpp:3219-3259 and 4614-4762, at network
 * level): runs engine command `command_index` again exactly as the last run
 * did (same kernel and tile, the input and its amax slots as the run left
 * them) with the int32 accumulators on, into acc ([N][OH][OW][OC] exact
 * sums of the quantized input times the int8 weights, acc_elements at
 * least N*OH*OW*OC), and, when slots is non-NULL, the input's per-16-channel
 * amax words (bit patterns of max|x| over each channel group, the max over
 * the slot copies: what the conv quantized with; slot_count >= C/16).  The
 * model's tensors and slots are not modified.  Returns 0 for commands that
 * are not per-tensor int8 convs (pg16, dynamic, fp16) or before a run. */
int aexrt_yolo_debug_conv_int8(AexrtYoloModel* model, uint32_t command_index, int32_t* acc,
                               uint64_t acc_elements, uint32_t* slots, uint32_t slot_count);
/* Logical dims of a value: out4 = {N, C, H, W} ({N, C, A, 1} for rank 3);
 * returns the rank, 0 when the value has no device storage. */
int aexrt_yolo_value_info(AexrtYoloModel* model, uint32_t value_id, uint32_t* out4);

/* native/aexrt.h:406-432 errors, timing and per-command profile events. */
const char* aexrt_yolo_get_last_error(AexrtYoloModel* model);
int aexrt_yolo_get_last_run_timing(AexrtYoloModel* model, AexrtYoloRunTiming* timing);
int aexrt_yolo_set_profiling(AexrtYoloModel* model, int enabled);
uint32_t aexrt_yolo_profile_event_count(AexrtYoloModel* model);
const char* aexrt_yolo_profile_event_label(AexrtYoloModel* model, uint32_t index);
double aexrt_yolo_profile_event_ms(AexrtYoloModel* model, uint32_t index);
/* Capture the run into a HIP graph (default on). */
int aexrt_yolo_set_graph_capture(AexrtYoloModel* model, int enabled);

/* native/aexrt.h:446-460 conv plan inspection and per-command override. */
uint32_t aexrt_yolo_conv_plan_count(AexrtYoloModel* model);
int aexrt_yolo_conv_plan_info(AexrtYoloModel* model, uint32_t index, AexrtConvPlanInfo* out_info);
int aexrt_yolo_override_conv_algorithm(AexrtYoloModel* model, uint32_t command_index, uint32_t algorithm_id);

/* native/aexrt.h:486 */
void aexrt_yolo_destroy(AexrtYoloModel* model);

#ifdef __cplusplus
}
#endif

#endif /* AEXRT_HIP_H_ */
