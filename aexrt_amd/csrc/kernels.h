// Launch interfaces of the gfx950 kernels (host side of the library).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace aexrt {

// Exact unsigned division by a launch constant d for n < 2^31: q = (umulhi(n,
// mul) + n) >> shift with l = ceil(log2 d), mul = 2^32 (2^l - d) / d + 1.
struct FastDiv {
    uint32_t mul;
    uint32_t shift;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t mul = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    return FastDiv{(uint32_t)mul, l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) { return (__umulhi(n, f.mul) + n) >> f.shift; }

// Largest byte span of one tensor view inside a conv launch: views are
// addressed with 32-bit buffer offsets; bigger batches are split into several
// launches by the host.
constexpr uint64_t kMaxViewBytes = 0x7FF00000ull;

// A (possibly striped) amax slot array: copy s of slot g at p[s * stride + g].
// Producers fold each workgroup's maxima into one copy, readers take the max
// over all copies.  p == nullptr: no slots.
struct SlotRef {
    uint32_t* p;
    uint32_t stripes;  // >= 1
    uint32_t stride;   // uint32 elements between copies
};

enum ConvFlags : int {
    kConvSilu = 1,      // SiLU after bias
    kConvResidual = 2,  // + residual tensor after the activation
    kConvOutF32 = 4,    // store fp32 instead of fp16
    kConvPg16 = 16,     // int8 with per-16-input-channel activation scales (pg16)
    kConvOutNchw = 32,  // pg16 only: dense NCHW output (the reference's layout)
    kConvDynamic = 64,  // int8 quantized per (position, 4 channels) in the kernel
};

// Views whose element (position m, channel c) sits at m * c_stride + c: the
// image stride is H*W*c_stride (every full-image view of an NHWC root) and,
// for kLinX, the conv is 1x1 stride 1 without padding.  Offsets then need
// no division; positions and strides must stay below 2^24 (24-bit multiply).
enum LinearViews : int {
    kLinX = 1,  // input pixel of position m at m * x_cstride
    kLinY = 2,  // output (and residual) of position m at m * y_cstride (r_cstride)
};

enum Loader : int {
    kLoaderNhwc = 0,     // fp16 NHWC activation view, C % 8 == 0
    kLoaderNchwF32 = 1,  // fp32 NCHW network input, c_real <= 4 channels read as C = 8 (zero padded)
    kLoaderPackedNc4 = 2,  // pg16 only: the reference's packed NC/4HW4 int8 words
};

// Kernel and tile of one conv launch.  kind 0: chosen by the heuristics;
// 1: implicit GEMM with tile (jn, pw, ksw); 2: halo-tile 3x3 with (jn, pw),
// tr x tc positions, cc channels per chunk and nw waves per block; 5: the
// 32x32-MFMA 3x3 with nq = jn, mq = pw, the halo fields and its wave groups
// minus one in ksw; 6: the streaming 1x1 with jq = jn, pq = pw and one tile
// per block (ksw).
struct ConvChoice {
    int kind = 0;
    int jn = 0, pw = 0, ksw = 0;
    int tr = 0, tc = 0, cc = 0;
    int nw = 4;  // halo: waves per block (4 or 8)
};

// One convolution launch.  Activation views address element (n, h, w, c) at
// n*nstride + (h*W + w)*cstride + c relative to their data pointer.
struct ConvParams {
    const void* x;
    int64_t x_nstride;
    int32_t x_cstride;
    int32_t loader;
    SlotRef x_slots;          // amax slots of the input channel range (int8 only)
    int32_t x_nslots;
    const void* w;            // [OCp][Kp], int8 or fp16
    int32_t Kp, OCp;
    const float* w_scale;     // [OC], int8 only
    const float* bias;        // [OC]
    void* y;
    int64_t y_nstride;
    int32_t y_cstride;
    SlotRef y_slots;          // amax slots of the output channels, p may be null
    const __half* res;        // residual view, same geometry as y
    int64_t r_nstride;
    int32_t r_cstride;
    int32_t* acc_out;         // optional int32 accumulators [M][OC] (int8)
    int N, H, W, C, OH, OW, OC, KH, KW, S, P;
    int c_real = 0;           // kLoaderNchwF32: channels present in memory (x_nstride = c_real*H*W)
    int lin = 0;              // kLinX / kLinY: view offsets linear in the position (set by the launcher)
    ConvChoice choice{};      // kernel / tile (kind 0: heuristics)
    int K, M;
    int flags;
    // host side only: a 1x1 fp16 conv applied to this conv's fp16 output in
    // the epilogue (its weights, bias, flags and output view; the input view
    // is this conv's output, which is then not stored).  Null: none.
    const struct ConvParams* fuse_1x1 = nullptr;
    // int8 1x1 convs on the streaming kernel: when yup is set, the output's
    // nearest 2x upsample (2 OH x 2 OW positions per image, NHWC view of
    // OC channels, e.g. a channel slice of a concat) is written there too,
    // and its amax folded into yup_slots.  Null: none.
    void* yup = nullptr;
    int64_t yup_nstride = 0;
    int32_t yup_cstride = 0;
    SlotRef yup_slots{};
    uint32_t yup_bytes = 0;  // filled in by the igemm launcher
    // int8 1x1 convs on the streaming kernel: input channels [xup_c0, xup_c0
    // + xup_cn) are read from xup, a map of H/2 x W/2 positions (NHWC view),
    // as its nearest 2x upsample, so that upsample is never stored (the input
    // view's memory for those channels is not read); xup_slots / xup_nslots:
    // that map's amax slots, read besides the input's.  Null: none.
    const void* xup = nullptr;
    int64_t xup_nstride = 0;
    int32_t xup_cstride = 0, xup_c0 = 0, xup_cn = 0;
    SlotRef xup_slots{};
    int32_t xup_nslots = 0;
    uint32_t xup_bytes = 0;  // filled in by the igemm launcher
    // filled in by the igemm launcher
    uint32_t x_bytes = 0, y_bytes = 0, r_bytes = 0;  // byte spans of the views
    uint32_t x_slot_bytes = 0;                       // byte span of the input slots
    int ntn = 1;                                     // output-channel tiles
    int npt = 1;                                     // position tiles
    int per = 1;                                     // position tiles per block
    FastDiv fd_ntn{}, fd_ohw{}, fd_ow{}, fd_c{}, fd_kw{}, fd_nit{}, fd_ns{};
};

// Per-wave tile of the igemm kernel: jn 16-channel subtiles x pw 16-position
// subtiles; ksw = the 4 waves of a block split the k steps of one tile.
struct ConvTile {
    int jn;
    int pw;
    bool ksw;
};
ConvTile choose_conv_tile(int M, int OC, int Kp);
// Forces every following igemm launch onto one tile shape (tuning and tests);
// (0, 0, 0) restores the automatic choice.  False for a shape that has no
// kernel instance.
bool set_conv_tile_override(int jn, int pw, int ksw);

// Kernel-name probe: while a probe is installed on the calling thread, the
// conv launchers (implicit GEMM, halo, stem, wide) write the kernel and tile
// they would launch into it and return hipSuccess without launching.
struct LaunchProbe {
    char name[96];
};
void set_launch_probe(LaunchProbe* probe);
LaunchProbe* launch_probe();
// Kernel and tile launch_conv_igemm(p, int8, ...) runs, as "family tile".
void conv_kernel_name(const ConvParams& p, bool int8, char* out, size_t n);

// Detect-head branch in one launch (conv_chain.hip): fp16 3x3 SiLU conv a,
// 3x3 SiLU conv b over a's output, 1x1 conv c over b's output (y), the two
// intermediate maps kept in LDS.  chain_shape_error: null when the three
// convs fit the kernel, else the reason.  chain_tile: the tile (rows tr x
// columns tc) the kernel runs (the given one when it fits; 0 x 0: chosen);
// false when none fits.
const char* chain_shape_error(const ConvParams& a, const ConvParams& b, const ConvParams& c);
bool chain_tile(const ConvParams& a, const ConvParams& b, const ConvParams& c, int& tr, int& tc);
hipError_t launch_conv_chain(const ConvParams& a, const ConvParams& b, const ConvParams& c, int tr, int tc,
                             hipStream_t stream);
// Two branches over one input (br0, br1: their a, b, c) in one launch on one
// tile (0 x 0: the one that fits the branch with more channels).
hipError_t launch_conv_chain2(const ConvParams* br0, const ConvParams* br1, int tr, int tc, hipStream_t stream);
// Tiles a chain launch can run on (br1 null: one branch; else both branches on
// the same tile), the largest first: whole map, halves, thirds, then 8x8 down
// to 3x3; up to cap (rows, columns) pairs written, their count returned.
int enumerate_chain_tiles(const ConvParams* br0, const ConvParams* br1, int* tr, int* tc, int cap);

// C2f bottleneck pair in one launch (conv_pair.h): conv a (3x3 s1 p1 SiLU,
// C -> C) then conv b (the same, + b.res when b.flags has kConvResidual) over
// a's output, which stays in LDS (t_out: optional dense NHWC copy of it;
// acc_a / b.acc_out: optional int32 sums, int8).  Bands of tr output rows
// (0: chosen).  int8: a grid barrier exchanges the intermediate's amax, so
// the whole grid must be resident (hipErrorInvalidConfiguration otherwise);
// sync: kPairSyncWords uint32 zero at launch (a generation word excepted),
// err: set to 1 if a barrier wait timed out.
constexpr int kPairSyncWordsHost = 512;
const char* pair_shape_error(const ConvParams& a, const ConvParams& b, bool int8);
int enumerate_pair_bands(const ConvParams& a, const ConvParams& b, bool int8, int* out, int cap);
hipError_t launch_conv_pair(const ConvParams& a, const ConvParams& b, bool int8, int tr, uint32_t* sync,
                            uint32_t* err, __half* t_out, int32_t* acc_a, hipStream_t stream);

// Implicit-GEMM conv (int8 or fp16 MFMA).  Requires C % 8 == 0, OC % 4 == 0,
// Kp % 64 == 0, OCp % 16 == 0 and 16-byte aligned views.
hipError_t launch_conv_igemm(const ConvParams& p, bool int8, hipStream_t stream);
// Every kernel/tile choice that can run conv p (implicit-GEMM tiles, and
// halo tiles for 3x3 convs), at most cap; returns the count.  Callers size
// their candidate arrays kMaxConvChoices, which no conv of the supported
// shapes reaches (a count equal to it means some were dropped).
constexpr int kMaxConvChoices = 256;
int enumerate_conv_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap);
int enumerate_halo_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap);
// Halo-tile 3x3 conv (pad 1, stride 1/2, C % 16 == 0) on one batch slice whose
// views fit 32-bit offsets: the input window of each position tile is staged
// (and quantized) once in LDS.  epi: 0 any flags, 1 SiLU -> fp16, 2 int8
// SiLU + residual -> fp16.  hipErrorNotSupported for other shapes.
hipError_t launch_conv_halo(const ConvParams& p, bool int8, int epi, hipStream_t stream);
// Halo kernel selection for 3x3 convs: mode 0 automatic, 1 never (implicit
// GEMM only), 2 forced tile (jn oc subtiles, pw position subtiles per wave,
// tr x tc output positions per tile, cc channels per chunk; a 3x3 conv the
// tile does not fit then fails).  False for a tile without a kernel instance.
bool set_conv3x3_halo(int mode, int jn, int pw, int tr, int tc, int cc);
// Wide-tile fp16 3x3 conv (choice kind 4): every output channel (49..80) in
// each wave, weights and input window streamed through LDS per channel chunk.
// epi 0 any flags / 1 SiLU; no residual or accumulator output.
int enumerate_wide_choices(const ConvParams& p, ConvChoice* out, int cap);
hipError_t launch_conv_wide(const ConvParams& p, int epi, hipStream_t stream);
// The tile forced by set_conv3x3_halo mode 4 (false: none).
bool forced_wide_choice(ConvChoice& c);
// 32x32-MFMA 3x3 conv (choice kind 5: jn = NQ 32-channel subtiles of the
// block, pw = MQ 32-position subtiles per wave, tr x tc positions per tile,
// cc channels per chunk; C % 16 == 0, weights of all chunks resident in LDS).
// epi as for the halo kernel.  hipErrorInvalidValue when the choice does not
// fit the conv.
int enumerate_m32_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap);
hipError_t launch_conv_m32(const ConvParams& p, bool int8, int epi, hipStream_t stream);
// Forces every 3x3 conv the kind-0 heuristics would run onto one m32 tile
// of nw (4 or 8) waves per block in ng (1, or 2 with 8 waves) wave groups
// (on = false: off).  False for a tile without a kernel instance.
bool set_conv3x3_m32(bool on, int mq, int nq, int tr, int tc, int cc, int nw, int ng);
bool forced_m32_choice(ConvChoice& c);
// Streaming 1x1 int8 conv (choice kind 6: jn = JQ 16-channel subtiles of the
// block, pw = PQ 16-position subtiles per wave; C % 16 == 0, positions evenly
// strided in both views, no residual): weights resident in LDS, every tile's
// input loaded at once and quantized once into an int8 LDS tile, the next
// tile in flight during the current one's MFMAs.  epi 0 any flags / 1 SiLU.
// hipErrorInvalidValue when the choice does not fit the conv.
// enumerate_s1x1_choices: the streaming tiles that fit conv p, at most cap.
int enumerate_s1x1_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap);
hipError_t launch_conv_s1x1(const ConvParams& p, bool int8, int epi, hipStream_t stream);
// Forces every int8 1x1 conv the kind-0 heuristics would run onto one
// streaming tile (on = false: off).  False for a tile without an instance.
bool set_conv1x1_stream(int mode, int jq, int pq);  // 0 off, 1 persistent, 2 one tile per block
bool forced_s1x1_choice(ConvChoice& c);
// Band kernel of the network's first conv (3x3 pad 1, stride 1/2, fp32 NCHW
// input of at most 3 channels read directly, fp16 SiLU output, OCp <= 64,
// W % 4 == 0): whole output rows per tile, one fp16 MFMA per 16 positions and
// 16 channels.  hipErrorNotSupported for other convs or when switched off.
hipError_t launch_conv_stem(const ConvParams& p, hipStream_t stream);
bool stem_shape_ok(const ConvParams& p);
int enumerate_stem_choices(const ConvParams& p, ConvChoice* out, int cap);
// Stem kernel selection: mode 0 automatic (band kernel when the conv fits),
// 1 never (halo-tile kernel), 2 forced band of tr output rows.
bool set_conv_stem(int mode, int tr);
// Input staging of the network's first conv: fp32 NCHW -> fp16 NHWC with the
// channels zero-padded to a multiple of 8 (one 16-byte store per pixel and
// 8 channels).  y has c_stride Cp = C rounded up to 8, dense.
hipError_t launch_nchw_f32_to_nhwc8(const float* x, __half* y, int N, int C, int HW, hipStream_t stream);

// Dynamic int8 conv (the reference's fallback for inputs of fewer than 4096
// elements): per (position, 4-channel group) scale computed in the kernel,
// v_dot4 int32 partials, fp32 dequant accumulation, + bias, SiLU (flags
// kConvSilu), fp16 residual (kConvResidual), fp32 output (kConvOutF32).
// w is the int8 [OCp][Kp] weight of the MFMA kernels (K = (ky, kx, c)).
struct DynConvParams {
    const __half* x;
    int64_t x_nstride;
    int32_t x_cstride;
    const int8_t* w;
    int32_t Kp;
    const float* w_scale;
    const float* bias;
    void* y;
    int64_t y_nstride;
    int32_t y_cstride;
    const __half* res;
    int64_t r_nstride;
    int32_t r_cstride;
    SlotRef y_slots;
    int N, H, W, C, OH, OW, OC, K, S;
    int flags;
};
hipError_t launch_conv_int8_dynamic(const DynConvParams& p, hipStream_t stream);

// fp32 direct conv on dense NCHW tensors (the reference's fp32 conv path):
// w [OC][C/G][KH][KW], bias [OC], y [N][OC][OH][OW]; acc = bias, += x*w in
// (channel, ky, kx) order without fused multiply-adds; silu: acc/(1+e^-acc).
struct F32ConvParams {
    const float* x;
    const float* w;
    const float* bias;
    float* y;
    int N, C, H, W, OC, OH, OW, KH, KW, SH, SW, PT, PL, DH, DW, G;
    int silu;
};
hipError_t launch_conv_f32(const F32ConvParams& p, hipStream_t stream);

// Winograd F(2x2,3x3), fp16 MFMA.  U is [16][OCp][Cp] fp16 (Cp = C rounded up
// to 32).  Same views/flags as ConvParams (w = U, Kp = Cp).
hipError_t launch_winograd_f2x2(const ConvParams& p, hipStream_t stream);

// ---- quantization / amax ---------------------------------------------------

// amax slots of an NHWC fp16 view: slots[g] |= max|x| over channels 16g..16g+15
// (atomicMax, caller clears).  C % 16 == 0.
hipError_t launch_amax_slots_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW,
                                  int C, SlotRef slots, hipStream_t stream);
// Strips of the reference's amax buffer over an NHWC fp16 view: max|x| of
// image n, group g folded into slots[(n * C/16 + g) / N], i.e. memory strip
// (n*C + 16g) / (16N) of the NCHW layout (slots[s] = the reference's
// amax[1 + s]).  C % 16 == 0; the caller clears the C/16 words.
hipError_t launch_amax_strips_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW, int C,
                                   uint32_t* slots, hipStream_t stream);
// The reference's amax buffer over an NCHW tensor (fp16 or fp32): slot 0 =
// whole tensor, slot 1+g = memory strip [g*16*N*HW, (g+1)*16*N*HW).
hipError_t launch_amax_strips_nchw(const void* x, bool f16, int N, int C, int HW, uint32_t* slots,
                                   hipStream_t stream);
// int8 NHWC (dense) from an fp16 NHWC view with the per-tensor amax of nslots slots.
hipError_t launch_quantize_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW, int C,
                                SlotRef slots, int nslots, int8_t* q, hipStream_t stream);
// The reference's NC/4HW4 pack (per-tensor slot 0, or per_group slots 1+icg/4).
hipError_t launch_quant_pack_nchw(const void* x, bool f16, int N, int C, int HW, const uint32_t* slots,
                                  bool per_group, uint32_t* packed, hipStream_t stream);

// pg16 int8 conv (native/aexrt_d3d12_runtime.cpp:4770-4923): 1x1 or 3x3,
// C % 16 == 0.  x_slots slot g = amax of input channel group g.  Loader
// kLoaderNhwc (fp16 view, quantized in the kernel per group) or
// kLoaderPackedNc4 (x = the reference's packed words); output an NHWC view
// (epilogue flags as the per-tensor kernels) or dense NCHW (kConvOutNchw).
hipError_t launch_conv_int8_pg16(const ConvParams& p, hipStream_t stream);
// The reference's fused pg16 amax + pack (RT:4083-4149) of an NCHW tensor:
// amax[1 + g] = max over image 0's channels 16g..16g+15, packed NC/4HW4.
hipError_t launch_quant_fused_pg16(const void* x, bool f16, int N, int C, int HW, uint32_t* packed,
                                   uint32_t* amax, hipStream_t stream);

// YOLO output0 postprocess (decode + filter, class-wise NMS, top-k) in one
// block; element (channel ch, anchor a) of output0 at out[ch * ch_stride + a *
// a_stride].  Writes count[0] = detections and dets[0 .. count) as x1, y1,
// x2, y2, score, class.  1 <= max_candidates <= kYoloMaxCandidates.  With
// levels, out is the raw Detect head (64 DFL bin logits, then class logits;
// anchors level by level, h x w each) and is decoded here; without, out is
// the decoded [4 (+1) + classes][anchors] tensor.
constexpr int kYoloMaxCandidates = 2048;
constexpr int kYoloMaxLevels = 4;
struct YoloLevels {
    int n;
    int h[kYoloMaxLevels], w[kYoloMaxLevels];
    float stride[kYoloMaxLevels];
};
hipError_t launch_yolo_decode_nms_topk(const float* out, int ch_stride, int a_stride, int anchors, int classes,
                                       int has_objectness, float conf, float iou, int max_candidates,
                                       int max_detections, float* dets, uint32_t* count, hipStream_t stream,
                                       const YoloLevels* levels = nullptr);

// ---- glue ------------------------------------------------------------------
hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream);
// dst view (channels [0,C)) = src view; amax slots of dst updated when non-null.
hipError_t launch_copy_nhwc(const __half* src, int64_t s_nstride, int32_t s_cstride, __half* dst,
                            int64_t d_nstride, int32_t d_cstride, int N, int HW, int C,
                            SlotRef dst_slots, hipStream_t stream);
hipError_t launch_maxpool_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y,
                               int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C,
                               int OH, int OW, int k, int s, int pad, SlotRef y_slots,
                               hipStream_t stream);
// SPPF's three chained 5x5 / s1 / p2 max pools of x in one pass: y1 = pool5(x),
// y2 = pool5(y1), y3 = pool5(y2), written to three views sharing strides, with
// their amax slots.  sppf_fits: the (H, W) plane fits the kernel's LDS.
bool sppf_fits(int H, int W);
hipError_t launch_sppf_maxpool_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y1, __half* y2,
                                    __half* y3, int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C,
                                    SlotRef s1, SlotRef s2, SlotRef s3, hipStream_t stream);
hipError_t launch_resize_nearest_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y,
                                      int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C,
                                      int OH, int OW, SlotRef y_slots, hipStream_t stream);
hipError_t launch_add_nhwc(const __half* a, int64_t a_nstride, int32_t a_cstride, const __half* b,
                           int64_t b_nstride, int32_t b_cstride, __half* y, int64_t y_nstride,
                           int32_t y_cstride, int N, int HW, int C, SlotRef y_slots, hipStream_t stream);
// fp32 NCHW <-> fp16 NHWC views.
hipError_t launch_nchw_f32_to_nhwc_f16(const float* x, __half* y, int64_t y_nstride, int32_t y_cstride,
                                       int N, int C, int HW, SlotRef y_slots, hipStream_t stream);
hipError_t launch_nhwc_to_nchw_f32(const void* x, bool f16, int64_t x_nstride, int32_t x_cstride, float* y,
                                   int N, int C, int HW, hipStream_t stream);

}  // namespace aexrt
