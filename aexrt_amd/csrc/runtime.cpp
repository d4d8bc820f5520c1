// Model runtime: executes a loaded .aexrt plan on the gfx950 kernels.
//
// Load time (once):
//   * parse and validate the engine (engine_loader.cpp);
//   * derive every value's logical dims from its producing command;
//   * fuse "conv -> residual add" pairs into the conv epilogue;
//   * place values in device memory: NHWC, fp16 (the network output fp32),
//     with every CONCAT input written straight into its slice of the concat
//     (channel or anchor axis), VIEW/ALIAS as offsets, so concats cost no
//     copy; each tensor keeps one amax slot per 16 channels;
//   * resolve each conv's kernel from the plan (int8 / Winograd / fp16, with
//     the reference's fail-closed fallback to the generic kernel,
//     native/aexrt_d3d12_runtime.cpp:9424-9500) and upload its weights in
//     the kernel's operand layout;
//   * build the launch list.
// Run time: one fill of the amax slots, then the launch list, captured once
// into a HIP graph and replayed (the reference's record-once / replay-every-
// frame structure, native/aexrt_d3d12_runtime.cpp:28758-29944).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "runtime.h"

struct AexrtDevice {
    int index = 0;
    hipDeviceProp_t props{};
    std::mutex mutex;
};

namespace aexrt {
namespace {

// Copies of the model's amax slot array: the workgroups of a layer spread
// their slot updates over this many cache lines (4 KB apart).
constexpr uint32_t kSlotStripes = 16;

struct Placement {
    bool valid = false;
    int root = -1;
    int64_t offset = 0;  // elements from the root base
    int64_t nstride = 0;
    int32_t cstride = 0;
    int slot = -1;       // first amax slot in the model's slot array
};

struct ValueInfo {
    int rank = 4;
    int N = 1, C = 1, H = 1, W = 1;  // rank 3 [N, C, A] stored as H = A, W = 1
    bool is_input = false, is_const = false, known = false;
    int producer = -1;
    std::vector<int> consumers;
    Placement pl;
    int redirect = -1;   // conv output fused into this value (residual add output)
    int cpad = 0;        // physical channels when zero-padded (network input)
    bool elided = false; // an fp16 conv output consumed only inside its producer's launch (never stored)
};

struct Root {
    int64_t elements = 0;
    bool f32 = false;
    int C = 0;
    int slot_base = -1;
    // an int8 conv reads a value of this root: its producers keep its amax
    // slots (slot updates of roots no int8 conv reads are skipped)
    bool slots_read = true;
    // every channel of the root is covered by a producer that folds into its
    // slots (false when a slice was placed at a channel offset or size that
    // is not a multiple of 16: int8 readers then take their own amax pass)
    bool slots_complete = true;
    size_t byte_offset = 0;
};

struct ConvState {
    bool is_conv = false;
    uint32_t planned = 0;
    uint32_t algorithm = 0;
    bool fused_residual = false;
    int residual_value = -1;
    int out_value = -1;       // value the conv writes (add output when fused)
    void* w = nullptr;
    float* scale = nullptr;
    float* bias = nullptr;
    bool pg16 = false;            // int8 with per-16-input-channel scales (plan flag 16)
    bool dynamic = false;         // int8 on an input of < 4096 elements: quantized per (position, 4 ch)
    uint32_t* strips = nullptr;   // pg16 at N > 1: the reference's strip amax of the input
    uint32_t* own_slots = nullptr;  // per-tensor int8 whose input slots are incomplete: its own amax pass
    uint64_t w_bytes = 0;         // bytes of w
    // a 1x1 fp16 conv applied in this 3x3 conv's epilogue (command index), or
    // the 3x3 conv this 1x1 conv is applied in; f2p: that 1x1's launch
    // parameters (its input is this conv's output, which is not stored)
    int fused_1x1 = -1, fused_into = -1;
    ConvParams f2p{};
    // a head branch run in one launch with this 3x3 conv first: the 3x3 conv
    // over its output (chain_b) and the 1x1 conv over that one's (chain_c)
    int chain_b = -1, chain_c = -1;
    // the chain launch's tile (rows x columns; 0 x 0: the largest that fits),
    // measured at load among the tiles the kernel offers
    int chain_tr = 0, chain_tc = 0;
    // C2f bottleneck superblock: this 3x3 conv and the 3x3 conv over its
    // output (pair_b) in one launch, the intermediate never stored; pair_a:
    // the first conv of the pair this one completes
    int pair_b = -1, pair_a = -1;
    // sibling pair (this conv first): weights and bias of both convs, rows of
    // this conv then the sibling's, built from the w of each named here
    void* w_pair = nullptr;
    float* bias_pair = nullptr;
    const void* pair_src[2] = {nullptr, nullptr};
};

struct Step {
    int cmd = -1;
    std::string label;
    std::function<hipError_t(hipStream_t)> launch;
    // memory roots the step reads / writes (all: every root and the slots)
    std::vector<int> reads, writes;
    bool all = false;
    // schedule: earlier steps it must follow, and its stream lane
    std::vector<int> deps;
    int lane = 0;
    bool signal = false;  // a later step on another lane waits for this one
    // conv steps: label = head + " kernel=" + family() + tail (the kernel that
    // runs can change after the step is built: measured tile choices)
    std::string head, tail;
    std::function<std::string()> family;
    // per-tensor int8 conv steps: the launch parameters as they run now (for
    // the accumulator debug tap)
    std::function<ConvParams()> conv_params;
    // a launch whose workgroups meet in a grid barrier (int8 superblock): never
    // concurrent with another such launch, which could hold the CUs it waits for
    bool grid_sync = false;
};

// Schedule of a network measured at load: sibling convs as one launch, lane
// count, head 1x1 convs fused into their 3x3 producers.
struct Schedule {
    int first = 1;        // sibling pairs in one launch
    int second = 1;       // lanes
    int fuse = 0;         // head 3x3 + 1x1 pairs in one launch: 0 none, else the pairs of mask
    uint32_t mask = 0;    // bit k: the k-th pair in command order (0 with fuse set: every pair)
    uint32_t chains = 0;  // bit k: the k-th head branch (3x3, 3x3, 1x1) in one launch
    uint32_t dual = 0;    // bit k: ... sharing its launch with the level's other branch
    int super = 0;        // C2f bottleneck superblocks on: bit 0 fp16 pairs, bit 1 int8 pairs
};

// Pairs a schedule fuses (bit k: the k-th head pair in command order).
uint32_t schedule_fuse_mask(const Schedule& s) { return s.fuse == 0 ? 0u : s.mask ? s.mask : ~0u; }

// A conv whose kernel choice is measured: its launch reads p (the choice
// can change after the step list is built).
struct TunedConv {
    int cmd = -1;
    std::string key;  // "cmd <index> <shape key>" of the measured choice
    size_t step = 0;
    ConvParams p{};
    bool int8 = false;
    std::vector<ConvChoice> cands;  // fastest first, as measured on their own
    bool done = false;              // choice measured in the running network (or read from the cache)
};

// Streams a captured graph spreads independent steps over.
constexpr int kLanes = 4;

// What the prepared step list does with the engine's commands, in the terms
// of the reference's counters (native/aexrt.h:307-385): commands folded into
// another launch, fusions, and convs per kernel family.
struct PlanStats {
    uint32_t skipped = 0;               // engine commands with no launch of their own
    uint32_t late_concat_conv1x1 = 0;   // concats placed in place and read whole by a 1x1 conv
    uint32_t paired_conv3x3 = 0;        // two 3x3 convs of one input computed by one launch
    uint32_t tail_residual = 0;         // residual adds in a conv epilogue
    uint32_t head_final_conv = 0;       // 1x1 convs applied in the preceding 3x3 conv's epilogue
    uint32_t conv1x1 = 0, spatial3x3 = 0, pack4_3x3 = 0, igemm3x3 = 0, igemm3x3_40 = 0, igemm3x3_20 = 0,
             igemm3x3_10 = 0;
    uint32_t exact_40_64x64 = 0, exact_20_64x64 = 0, exact_10_128x128 = 0, exact_20_128x64 = 0,
             exact_10_256x64 = 0;
    uint32_t native_fp16 = 0;
    uint32_t c2f_superblocks = 0;       // C2f bottleneck pairs run as one launch
};

// A CONCAT input that could not be placed inside its concat: copied there.
struct CopyJob {
    int cmd;
    int src;
    Placement dst;
};

const char* kind_name(uint32_t k) {
    static const char* names[] = {"?", "CONV", "CONV_SILU", "CONCAT_CONV1X1", "VIEW", "ALIAS", "SLICE", "CONCAT",
                                  "RESIZE", "MAXPOOL", "UNARY", "BINARY", "MATMUL", "TRANSPOSE", "SOFTMAX"};
    return k < 15 ? names[k] : "?";
}

const char* algorithm_name(uint32_t a) {
    if (a == 51) return "int8_mfma_1x1";
    if (a == 52) return "int8_mfma_3x3";
    if (a == 53) return "int8_mfma_3x3s2";
    if (a == 40 || a == 46) return "winograd_f2x2_fp16_mfma";
    return "fp16_mfma_igemm";
}

}  // namespace
}  // namespace aexrt

using namespace aexrt;

struct AexrtYoloModel {
    AexrtDevice* device = nullptr;
    Engine eng;
    std::vector<ValueInfo> vals;
    std::vector<Root> roots;
    std::vector<ConvState> convs;
    // per command: the sibling conv whose output is placed right after this
    // conv's output channels in one root (one launch computes both), or -1
    std::vector<int> sibling;
    bool merge_siblings = true;  // sibling pairs run as one launch (measured at load)
    // head 3x3 + 1x1 pairs that run as one launch (bit k: the k-th pair in command
    // order; measured at load), and every such pair of the plan (3x3, 1x1 command)
    uint32_t fuse_mask = 0;
    std::vector<std::pair<int, int>> fuse_pairs;
    // head branches (3x3 SiLU, 3x3 SiLU, 1x1 commands) that can run in one
    // launch, and those that do (bit k: the k-th in command order; measured
    // at load per head level)
    std::vector<std::array<int, 3>> chains;
    uint32_t chain_mask = 0;
    uint32_t chain_dual = 0;  // branches of chain_mask that share a launch with another over their input
    std::vector<Step> steps;
    std::vector<CopyJob> copies;
    // C2f bottleneck superblocks (AEXRT_HIP_C2F_SUPERBLOCK=1): their grid
    // barriers' sync words (cleared every run) and the barrier-timeout word
    uint32_t superblock_mask = 0;  // bit 0: fp16 pairs as superblocks, bit 1: int8 pairs
    // per command: a nearest 2x resize folded into the int8 1x1 conv that
    // produces its input (the conv's entry names the resize, the resize's
    // the conv); -1: none
    std::vector<int> up_fold;
    // per command: a nearest 2x resize whose output (a concat slice) the
    // int8 1x1 conv reading the concat reads from the resize's input instead,
    // so the upsample is never stored (the conv's entry names the resize, the
    // resize's the conv); -1: none
    std::vector<int> up_read;
    uint32_t* pair_sync = nullptr;
    int n_pair_sync = 0;
    uint32_t* pair_err = nullptr;
    std::vector<void*> allocations;
    uint8_t* arena = nullptr;
    uint32_t* slots = nullptr;
    int nslots = 0;
    uint32_t slot_stride = 0;  // uint32 elements between the slot copies
    float* input_dev = nullptr;
    float* input_host = nullptr;
    bool input_needs_nhwc = false;
    bool input_nchw_direct = false;  // the input's convs read the fp32 NCHW tensor themselves
    bool autotune = true;            // measure every conv's kernel/tile choices at load
    bool tune_log = false;           // print each measured choice (AEXRT_HIP_TUNE_LOG=1)
    std::map<std::string, ConvChoice> tuned;  // conv shape -> measured choice
    std::map<std::string, std::vector<ConvChoice>> tuned_top;  // conv shape -> fastest candidates
    std::vector<std::unique_ptr<TunedConv>> tunables;         // convs of the step list with measured choices
    // chain launches of the step list: first branch's command, the other
    // branch's (-1: one branch), the step, the key of its tile choice
    struct ChainStep {
        size_t ci = 0;
        int partner = -1;
        size_t step = 0;
        std::string key;
        bool done = false;
    };
    std::vector<ChainStep> chain_steps;
    // "cmd <index> <shape key>" -> choice measured in the network (the shape key
    // keeps a cached choice from applying to the same command at another batch)
    std::map<std::string, ConvChoice> refined;
    // "schedule <input dims> <commands>" -> schedule measured at load
    std::map<std::string, Schedule> schedules;
    std::string tune_cache;                    // AEXRT_HIP_TUNE_CACHE file, empty: none
    hipStream_t lane_stream[kLanes] = {};      // capture-time streams of lanes 1..kLanes-1
    int n_lanes = 1;                           // lanes the schedule uses (measured at load)
    // how steps are put on lanes: 0 the dependency rule, 1 list scheduling over
    // step_ms, 2 lane_plan (a plan measured before, read from the tune cache)
    int lane_policy = 0;
    int lane_policy_forced = -1;              // AEXRT_HIP_LIST_SCHEDULE=0 / 1, else -1
    std::vector<float> step_ms;               // per step: its time in the network on one lane
    std::string lane_plan;                    // per step: its lane as a digit
    // "lanes <input dims> <commands>" -> lane plan measured at load (list scheduling kept)
    std::map<std::string, std::string> lane_plans;
    std::vector<hipEvent_t> step_events;      // per step, recorded when a step signals
    std::vector<hipEvent_t> lane_events;      // fork / join events of the captures
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    bool graph_valid = false;
    bool use_graph = true;
    bool profile = false;
    std::vector<std::string> prof_labels;
    std::vector<double> prof_ms;
    AexrtYoloRunTiming timing{};
    aexrt::PlanStats stats{};
    std::string last_error;
    bool executable = false;
    // YOLO postprocess of output0 (decode + filter, NMS, top-k)
    bool post_ok = false;
    bool post_dfl = false;            // output0 is the raw Detect head (DFL bins + class logits)
    aexrt::YoloLevels post_levels{};
    float* dets_dev = nullptr;        // [max_detections][6]
    uint32_t* det_count_dev = nullptr;
    std::mutex mutex;
};

namespace aexrt {
namespace {

bool fail(AexrtYoloModel* m, const std::string& msg) {
    if (m) m->last_error = msg;
    set_error(msg);
    return false;
}

void* dev_alloc(AexrtYoloModel* m, size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
    m->allocations.push_back(p);
    return p;
}

// ---- value dims ------------------------------------------------------------------
bool infer_dims(AexrtYoloModel* m) {
    Engine& e = m->eng;
    auto& V = m->vals;
    V.assign(e.values.size(), ValueInfo{});
    for (size_t i = 0; i < e.values.size(); ++i) {
        const EngineValue& v = e.values[i];
        V[i].is_input = (v.flags & 1u) != 0;
        V[i].is_const = (v.flags & 2u) != 0;
        if (V[i].is_input) {
            V[i].N = (int)v.shape4[0];
            V[i].C = (int)v.shape4[1];
            V[i].H = (int)v.shape4[2];
            V[i].W = (int)v.shape4[3];
            V[i].known = true;
        }
    }
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        ValueInfo& o = V[c.output];
        if (o.producer >= 0) return fail(m, "value " + std::to_string(c.output) + " is produced twice");
        o.producer = (int)ci;
        for (uint32_t in : c.inputs) V[in].consumers.push_back((int)ci);
        const std::vector<uint32_t>& p = c.params;
        auto need_in = [&](size_t k) -> ValueInfo* {
            if (k >= c.inputs.size()) return nullptr;
            ValueInfo* x = &V[c.inputs[k]];
            return x->known ? x : nullptr;
        };
        switch (c.kind) {
            case kCmdConv:
            case kCmdConvSilu: {
                ValueInfo* x = need_in(0);
                if (!x || p.size() < 16 || c.inputs.size() < 3)
                    return fail(m, "command " + std::to_string(ci) + ": malformed conv");
                if ((int)p[0] != x->N || (int)p[1] != x->C || (int)p[2] != x->H || (int)p[3] != x->W || x->rank != 4)
                    return fail(m, "command " + std::to_string(ci) + ": conv descriptor does not match its input");
                o.N = (int)p[0];
                o.C = (int)p[4];
                o.H = (int)p[5];
                o.W = (int)p[6];
                break;
            }
            case kCmdView: {
                ValueInfo* x = need_in(0);
                if (!x || p.size() < 2 || x->rank != 4) return fail(m, "command " + std::to_string(ci) + ": bad VIEW");
                const uint64_t trailing = uint64_t(x->H) * x->W;
                if (p[0] % trailing || p[1] % trailing || (p[0] + p[1]) / trailing > uint64_t(x->C))
                    return fail(m, "command " + std::to_string(ci) + ": VIEW is not a channel slice");
                o.N = x->N;
                o.C = (int)(p[1] / trailing);
                o.H = x->H;
                o.W = x->W;
                break;
            }
            case kCmdAlias: {
                ValueInfo* x = need_in(0);
                if (!x) return fail(m, "command " + std::to_string(ci) + ": bad ALIAS");
                const uint32_t* s4 = e.values[c.output].shape4;
                if (x->rank == 4 && (int)s4[0] == x->N && (int)s4[1] == x->C && (int)s4[2] == x->H &&
                    (int)s4[3] == x->W) {
                    o.rank = 4;
                    o.N = x->N, o.C = x->C, o.H = x->H, o.W = x->W;
                } else if (x->rank == 4 && s4[0] == 1 && (int)s4[1] == x->N && (int)s4[2] == x->C &&
                           (int)s4[3] == x->H * x->W) {
                    o.rank = 3;
                    o.N = x->N, o.C = x->C, o.H = x->H * x->W, o.W = 1;
                } else {
                    return fail(m, "command " + std::to_string(ci) + ": only [N,C,H,W]->[N,C,H*W] reshapes are supported");
                }
                break;
            }
            case kCmdConcat: {
                if (p.size() < 8 || c.inputs.empty()) return fail(m, "command " + std::to_string(ci) + ": bad CONCAT");
                const uint32_t rank = p[1], axis = p[2];
                const uint32_t* s4 = &p[4];
                if (rank == 4) {
                    o.rank = 4, o.N = (int)s4[0], o.C = (int)s4[1], o.H = (int)s4[2], o.W = (int)s4[3];
                    if (axis != 1) return fail(m, "command " + std::to_string(ci) + ": rank-4 CONCAT only along channels");
                } else if (rank == 3) {
                    o.rank = 3, o.N = (int)s4[1], o.C = (int)s4[2], o.H = (int)s4[3], o.W = 1;
                    if (axis != 2 && axis != 3) return fail(m, "command " + std::to_string(ci) + ": rank-3 CONCAT only along C or A");
                } else {
                    return fail(m, "command " + std::to_string(ci) + ": CONCAT rank must be 3 or 4");
                }
                int sum = 0;
                for (size_t k = 0; k < c.inputs.size(); ++k) {
                    ValueInfo* x = need_in(k);
                    if (!x || x->rank != (int)rank || x->N != o.N)
                        return fail(m, "command " + std::to_string(ci) + ": CONCAT input mismatch");
                    const bool along_c = (rank == 4 && axis == 1) || (rank == 3 && axis == 2);
                    if (along_c) {
                        if (x->H != o.H || x->W != o.W) return fail(m, "command " + std::to_string(ci) + ": CONCAT dims");
                        sum += x->C;
                    } else {
                        if (x->C != o.C) return fail(m, "command " + std::to_string(ci) + ": CONCAT dims");
                        sum += x->H;
                    }
                }
                const bool along_c = (rank == 4 && axis == 1) || (rank == 3 && axis == 2);
                if (sum != (along_c ? o.C : o.H)) return fail(m, "command " + std::to_string(ci) + ": CONCAT sizes");
                break;
            }
            case kCmdMaxpool: {
                ValueInfo* x = need_in(0);
                if (!x || p.size() < 13 || p[6] != p[7] || p[8] != p[9] || p[10] != p[11] || p[12] != 1)
                    return fail(m, "command " + std::to_string(ci) + ": unsupported MAXPOOL");
                o.N = (int)p[0], o.C = (int)p[1], o.H = (int)p[4], o.W = (int)p[5];
                if (x->rank != 4 || x->N != o.N || x->C != o.C || x->H != (int)p[2] || x->W != (int)p[3])
                    return fail(m, "command " + std::to_string(ci) + ": MAXPOOL input mismatch");
                // the output is what the pooling window yields (floor mode), so
                // the kernel never writes past the output root
                const int64_t k = p[6], st = p[8], pad = p[10];
                if (k < 1 || st < 1 || 2 * pad > k || (int64_t)x->H + 2 * pad < k || (int64_t)x->W + 2 * pad < k ||
                    o.H != ((int64_t)x->H + 2 * pad - k) / st + 1 || o.W != ((int64_t)x->W + 2 * pad - k) / st + 1)
                    return fail(m, "command " + std::to_string(ci) + ": MAXPOOL output dims do not follow the window");
                break;
            }
            case kCmdResize: {
                ValueInfo* x = need_in(0);
                if (!x || p.size() < 6) return fail(m, "command " + std::to_string(ci) + ": bad RESIZE");
                o.N = (int)p[0], o.C = (int)p[1], o.H = (int)p[4], o.W = (int)p[5];
                // the kernel runs over the input's images and channels into an
                // output root sized from these params: they must agree
                if (x->rank != 4 || (int)p[0] != x->N || (int)p[1] != x->C || (int)p[2] != x->H || (int)p[3] != x->W ||
                    o.H < 1 || o.W < 1)
                    return fail(m, "command " + std::to_string(ci) + ": RESIZE params do not match its input");
                break;
            }
            case kCmdBinary: {
                ValueInfo* a = need_in(0);
                ValueInfo* b = need_in(1);
                if (!a || !b || p.size() < 2 || p[1] != 0)
                    return fail(m, "command " + std::to_string(ci) + ": only BINARY add is supported");
                if (a->rank != 4 || b->rank != 4 || a->N != b->N || a->C != b->C || a->H != b->H || a->W != b->W)
                    return fail(m, "command " + std::to_string(ci) + ": BINARY add needs equal shapes");
                o.N = a->N, o.C = a->C, o.H = a->H, o.W = a->W;
                break;
            }
            default:
                return fail(m, "command " + std::to_string(ci) + ": kind " + kind_name(c.kind) +
                                   " is not supported by the HIP runtime");
        }
        o.known = true;
    }
    if (!V[e.manifest.output_value].known) return fail(m, "output value is never produced");
    return true;
}

// ---- residual fusion ----------------------------------------------------------------
void fuse_residuals(AexrtYoloModel* m) {
    Engine& e = m->eng;
    auto& V = m->vals;
    m->convs.assign(e.commands.size(), ConvState{});
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        if (c.kind == kCmdConv || c.kind == kCmdConvSilu) {
            m->convs[ci].is_conv = true;
            m->convs[ci].out_value = (int)c.output;
        }
    }
    for (size_t ai = 0; ai < e.commands.size(); ++ai) {
        const EngineCommand& a = e.commands[ai];
        if (a.kind != kCmdBinary) continue;
        for (int k = 1; k >= 0; --k) {
            const uint32_t r = a.inputs[k], other = a.inputs[1 - k];
            const int pc = V[r].producer;
            if (pc < 0 || !m->convs[pc].is_conv || V[r].consumers.size() != 1 ||
                r == e.manifest.output_value || m->convs[pc].fused_residual)
                continue;
            if (V[other].producer >= pc || V[other].is_const) continue;  // must exist before the conv runs
            if (V[other].is_input) continue;
            m->convs[pc].fused_residual = true;
            m->convs[pc].residual_value = (int)other;
            m->convs[pc].out_value = (int)a.output;
            V[r].redirect = (int)a.output;
            break;
        }
    }
}

bool is_f32(AexrtYoloModel* m, int v);
AexrtConv2DDesc desc_of(const EngineCommand& c);

// The last two convs of each YOLO head branch, 3x3 SiLU then a 1x1 of its
// output (its only consumer), both fp16: the 1x1 runs in the 3x3 conv's
// epilogue on the 32x32-MFMA kernel (every 3x3 output channel of a position
// in one block, so at most 96), and the 3x3 output is never stored.
// Fuses the pairs of m->fuse_mask (clears the others) and lists every pair the
// plan has in m->fuse_pairs; returns their number.
int fuse_head_1x1(AexrtYoloModel* m) {
    const Engine& e = m->eng;
    auto& V = m->vals;
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        ConvState& cs = m->convs[ci];
        if (cs.fused_1x1 >= 0) V[e.commands[ci].output].elided = false;
        cs.fused_1x1 = cs.fused_into = -1;
    }
    int pairs = 0;
    m->fuse_pairs.clear();
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        ConvState& cs = m->convs[ci];
        const EngineCommand& c = e.commands[ci];
        if (!cs.is_conv || c.kind != kCmdConvSilu || cs.fused_residual || cs.pg16 || cs.fused_into >= 0 ||
            is_int8_algorithm(cs.algorithm) || is_winograd_algorithm(cs.algorithm) || m->sibling[ci] >= 0)
            continue;
        const AexrtConv2DDesc d = desc_of(c);
        const ValueInfo& x = V[c.inputs[0]];
        const ValueInfo& y = V[c.output];
        if (d.kernel_h != 3 || d.kernel_w != 3 || d.stride_h != 1 || d.pad_top != 1 || d.in_channels % 16 ||
            d.out_channels > 96 || x.is_input || y.consumers.size() != 1 || y.redirect >= 0 || y.rank != 4 ||
            c.output == e.manifest.output_value)
            continue;
        bool paired = false;
        for (int s2 : m->sibling) paired = paired || s2 == (int)ci;
        if (paired) continue;
        const int cj = y.consumers[0];
        const ConvState& cn = m->convs[cj];
        const EngineCommand& n = e.commands[cj];
        if (!cn.is_conv || cn.fused_residual || cn.pg16 || is_int8_algorithm(cn.algorithm) ||
            is_winograd_algorithm(cn.algorithm) || n.inputs[0] != c.output || m->sibling[cj] >= 0)
            continue;
        const AexrtConv2DDesc d2 = desc_of(n);
        if (d2.kernel_h != 1 || d2.kernel_w != 1 || d2.stride_h != 1 || d2.pad_top != 0 || d2.out_channels > 96 ||
            d2.out_channels % 8)
            continue;
        m->fuse_pairs.emplace_back((int)ci, cj);
        const int k = pairs++;
        if (k >= 32 || !((m->fuse_mask >> k) & 1u)) continue;
        cs.fused_1x1 = cj;
        m->convs[cj].fused_into = (int)ci;
        V[c.output].elided = true;
    }
    return pairs;
}

// Head branches that can run in one launch: a fp16 3x3 stride-1 SiLU conv
// whose output only a second such conv reads, whose output only a 1x1 fp16
// conv reads, every channel count <= 96.  Lists them in m->chains; those of
// m->chain_mask take over their convs (the two intermediates are not stored,
// and a head pair fused by fuse_head_1x1 inside such a branch is undone).
// Returns the number of branches.
int setup_chains(AexrtYoloModel* m) {
    const Engine& e = m->eng;
    auto& V = m->vals;
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        ConvState& cs = m->convs[ci];
        if (cs.chain_b >= 0) {
            V[e.commands[ci].output].elided = false;
            V[e.commands[cs.chain_b].output].elided = m->convs[cs.chain_b].fused_1x1 >= 0;
        }
        cs.chain_b = cs.chain_c = -1;
    }
    m->chains.clear();
    auto fp16_conv = [&](size_t ci, uint32_t k) {
        const ConvState& cs = m->convs[ci];
        const EngineCommand& c = e.commands[ci];
        if (!cs.is_conv || cs.fused_residual || cs.pg16 || is_int8_algorithm(cs.algorithm) ||
            is_winograd_algorithm(cs.algorithm))
            return false;
        const AexrtConv2DDesc d = desc_of(c);
        const ValueInfo& x = V[c.inputs[0]];
        return d.kernel_h == k && d.kernel_w == k && d.stride_h == 1 && d.stride_w == 1 && d.pad_top == k / 2 &&
               d.out_channels <= 96 && !x.is_input && (k == 1 || (c.kind == kCmdConvSilu && d.in_channels % 16 == 0));
    };
    auto only_consumer = [&](size_t ci) {
        const ValueInfo& y = V[e.commands[ci].output];
        if (y.consumers.size() != 1 || y.redirect >= 0 || y.rank != 4 || e.commands[ci].output == e.manifest.output_value)
            return -1;
        const int cj = y.consumers[0];
        return e.commands[cj].inputs[0] == e.commands[ci].output ? cj : -1;
    };
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        if (!fp16_conv(ci, 3)) continue;
        const int cb = only_consumer(ci);
        if (cb < 0 || !fp16_conv((size_t)cb, 3)) continue;
        const int cc = only_consumer((size_t)cb);
        if (cc < 0 || !fp16_conv((size_t)cc, 1) || m->convs[cb].fused_residual) continue;
        bool sib_b = false;  // the second conv must not be half of a sibling pair
        for (size_t k = 0; k < m->sibling.size(); ++k)
            sib_b = sib_b || m->sibling[k] == cb || (k == (size_t)cb && m->sibling[k] >= 0);
        if (sib_b) continue;
        const int k = (int)m->chains.size();
        m->chains.push_back({(int)ci, cb, cc});
        if (k >= 32 || !((m->chain_mask >> k) & 1u)) continue;
        ConvState& cs = m->convs[ci];
        ConvState& bs = m->convs[cb];
        if (bs.fused_1x1 >= 0) {  // the branch's 1x1 pair: now part of the branch
            m->convs[bs.fused_1x1].fused_into = -1;
            bs.fused_1x1 = -1;
        }
        cs.chain_b = cb;
        cs.chain_c = cc;
        V[e.commands[ci].output].elided = true;
        V[e.commands[cb].output].elided = true;
    }
    return (int)m->chains.size();
}

// C2f bottlenecks whose two 3x3 convs can run as one superblock launch: a
// 3x3 stride-1 SiLU conv C -> C (int8 per-tensor or fp16, 32 <= C <= 128 in
// steps of 32) whose output only a second such conv of the same arithmetic
// reads, that second conv taking the first one's input as its fused residual
// or no residual.  The pairs of the arithmetics in m->superblock_mask (bit 0
// fp16, bit 1 int8) are marked (their intermediate is then never stored);
// returns the arithmetics the plan has pairs of, as such bits.
int setup_pairs(AexrtYoloModel* m) {
    const Engine& e = m->eng;
    auto& V = m->vals;
    int n = 0;
    auto conv3 = [&](size_t ci, int C) {
        const ConvState& cs = m->convs[ci];
        const EngineCommand& c = e.commands[ci];
        if (!cs.is_conv || c.kind != kCmdConvSilu || cs.pg16 || cs.dynamic || cs.own_slots ||
            is_winograd_algorithm(cs.algorithm) || cs.fused_1x1 >= 0 || cs.fused_into >= 0 || cs.chain_b >= 0 ||
            cs.chain_c >= 0 || m->sibling[ci] >= 0)
            return false;
        const AexrtConv2DDesc d = desc_of(c);
        return d.kernel_h == 3 && d.kernel_w == 3 && d.stride_h == 1 && d.pad_top == 1 && d.in_channels == (uint32_t)C &&
               d.out_channels == (uint32_t)C && d.in_h == d.out_h && d.in_w == d.out_w && C % 32 == 0 && C <= 128;
    };
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        ConvState& cs = m->convs[ci];
        if (cs.pair_b >= 0) V[e.commands[ci].output].elided = false;
        cs.pair_a = cs.pair_b = -1;
    }
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        ConvState& cs = m->convs[ci];
        if (!cs.is_conv || cs.fused_residual || cs.pair_a >= 0) continue;
        const int C = (int)desc_of(c).in_channels;
        if (!conv3(ci, C)) continue;
        const ValueInfo& t = V[c.output];
        const ValueInfo& x = V[c.inputs[0]];
        if (t.consumers.size() != 1 || t.redirect >= 0 || c.output == e.manifest.output_value || x.is_input ||
            !x.pl.valid)
            continue;
        const int cj = t.consumers[0];
        ConvState& bs = m->convs[cj];
        if (e.commands[cj].inputs[0] != c.output || !conv3((size_t)cj, C) ||
            is_int8_algorithm(bs.algorithm) != is_int8_algorithm(cs.algorithm))
            continue;
        if (bs.fused_residual && bs.residual_value != (int)c.inputs[0]) continue;
        if (is_int8_algorithm(cs.algorithm) && !m->roots[x.pl.root].slots_complete) continue;
        const int bit = is_int8_algorithm(cs.algorithm) ? 2 : 1;
        n |= bit;
        if (!(m->superblock_mask & (uint32_t)bit)) continue;
        cs.pair_b = cj;
        bs.pair_a = (int)ci;
        V[c.output].elided = true;
    }
    return n;
}

bool is_fused_add(AexrtYoloModel* m, size_t ci) {
    const EngineCommand& c = m->eng.commands[ci];
    if (c.kind != kCmdBinary) return false;
    for (uint32_t in : c.inputs)
        if (m->vals[in].redirect == (int)c.output) return true;
    return false;
}

// Only int8 convs read amax slots (the per-tensor scale of their input): the
// producers of every other root skip their slot updates, which are atomics
// on a few shared cache lines.
void mark_slot_readers(AexrtYoloModel* m) {
    for (Root& r : m->roots) r.slots_read = false;
    for (size_t ci = 0; ci < m->eng.commands.size(); ++ci) {
        const ConvState& cs = m->convs[ci];
        if (!cs.is_conv || !is_int8_algorithm(cs.algorithm) || cs.dynamic) continue;
        const ValueInfo& x = m->vals[m->eng.commands[ci].inputs[0]];
        if (x.pl.valid && x.pl.root >= 0) m->roots[x.pl.root].slots_read = true;
    }
}

// ---- placement ------------------------------------------------------------------------
int new_root(AexrtYoloModel* m, int v, bool f32) {
    ValueInfo& x = m->vals[v];
    const int C = x.cpad > x.C ? x.cpad : x.C;
    Root r;
    r.elements = int64_t(x.N) * x.H * x.W * C;
    r.f32 = f32;
    r.C = C;
    if (!f32 && C % 16 == 0 && C / 16 <= 128) {
        r.slot_base = m->nslots;
        m->nslots += C / 16;
    }
    m->roots.push_back(r);
    x.pl.valid = true;
    x.pl.root = (int)m->roots.size() - 1;
    x.pl.offset = 0;
    x.pl.cstride = C;
    x.pl.nstride = int64_t(x.H) * x.W * C;
    x.pl.slot = r.slot_base;
    return x.pl.root;
}

bool writer_kind(uint32_t k) {
    return k == kCmdConv || k == kCmdConvSilu || k == kCmdMaxpool || k == kCmdResize || k == kCmdBinary ||
           k == kCmdConcat;
}

bool same_placement(const Placement& a, const Placement& b) {
    return a.valid && b.valid && a.root == b.root && a.offset == b.offset && a.nstride == b.nstride &&
           a.cstride == b.cstride && a.slot == b.slot;
}

// Tries to make value t (C_t channels) live at `pl` (already shifted for t).
bool try_place(AexrtYoloModel* m, int t, const Placement& pl) {
    ValueInfo& x = m->vals[t];
    if (x.is_input || x.is_const) return false;
    if (x.pl.valid) return same_placement(x.pl, pl);
    if (x.producer < 0) return false;
    const uint32_t k = m->eng.commands[x.producer].kind;
    if (!writer_kind(k)) return false;
    if (k == kCmdBinary && is_fused_add(m, x.producer)) {
        // a fused add is written by its conv; fine as long as nothing else is special
    }
    x.pl = pl;
    return true;
}

AexrtConv2DDesc desc_of(const EngineCommand& c);

// A conv that can share a launch with a sibling: fp16 direct kernels (every
// plan id other than int8 and Winograd runs them from [OCp][Kp] weights), no
// fused residual, its own output not placed yet (not a concat member, not
// the network output), 16-channel aligned.
bool sibling_candidate(AexrtYoloModel* m, size_t ci) {
    const Engine& e = m->eng;
    const ConvState& cs = m->convs[ci];
    if (!cs.is_conv || cs.fused_residual || cs.pg16 || is_int8_algorithm(cs.algorithm) ||
        is_winograd_algorithm(cs.algorithm))
        return false;
    const EngineCommand& c = e.commands[ci];
    const ValueInfo& y = m->vals[c.output];
    const ValueInfo& x = m->vals[c.inputs[0]];
    return (c.kind == kCmdConv || c.kind == kCmdConvSilu) && !y.pl.valid && y.redirect < 0 && y.rank == 4 &&
           c.output != e.manifest.output_value && !x.is_input && y.C % 16 == 0;
}

// Two fp16 convs of one input with the same geometry and epilogue (the box
// and class branches of a detect head level) write adjacent channel ranges
// of one root: a single launch with the output channels of both computes
// them (every output channel is its own dot product, so the values are
// those of two launches up to the kernel choice).
void place_sibling_convs(AexrtYoloModel* m) {
    const Engine& e = m->eng;
    auto& V = m->vals;
    m->sibling.assign(e.commands.size(), -1);
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        if (!sibling_candidate(m, ci)) continue;
        const EngineCommand& a = e.commands[ci];
        const AexrtConv2DDesc da = desc_of(a);
        for (size_t cj = ci + 1; cj < e.commands.size(); ++cj) {
            const EngineCommand& b = e.commands[cj];
            if (b.kind != a.kind || b.inputs[0] != a.inputs[0] || !sibling_candidate(m, cj)) continue;
            AexrtConv2DDesc db = desc_of(b);
            db.out_channels = da.out_channels;
            if (std::memcmp(&da, &db, sizeof(da)) != 0) continue;
            const ValueInfo& ya = V[a.output];
            const int ca = ya.C, cb = V[b.output].C;
            Root r;
            r.C = ca + cb;
            r.elements = int64_t(ya.N) * ya.H * ya.W * r.C;
            if (r.C / 16 <= 128) {
                r.slot_base = m->nslots;
                m->nslots += r.C / 16;
            }
            m->roots.push_back(r);
            const int root = (int)m->roots.size() - 1;
            for (int k = 0; k < 2; ++k) {
                ValueInfo& y = V[k ? b.output : a.output];
                y.pl.valid = true;
                y.pl.root = root;
                y.pl.offset = k ? ca : 0;
                y.pl.cstride = r.C;
                y.pl.nstride = int64_t(y.H) * y.W * r.C;
                y.pl.slot = r.slot_base >= 0 ? r.slot_base + (k ? ca / 16 : 0) : -1;
            }
            m->sibling[ci] = (int)cj;
            break;
        }
    }
}

bool plan_memory(AexrtYoloModel* m, std::vector<CopyJob>& copies) {
    Engine& e = m->eng;
    auto& V = m->vals;
    const uint32_t out_v = e.manifest.output_value;
    // the network output lives in an fp32 root
    {
        int v = (int)out_v;
        while (V[v].producer >= 0 && e.commands[V[v].producer].kind == kCmdAlias) v = (int)e.commands[V[v].producer].inputs[0];
        new_root(m, v, true);
        if (v != (int)out_v) V[out_v].pl = V[v].pl;
    }
    for (int ci = (int)e.commands.size() - 1; ci >= 0; --ci) {
        const EngineCommand& c = e.commands[ci];
        if (c.kind == kCmdAlias) {
            // an aliased value that got placed lends its placement to the source
            ValueInfo& o = V[c.output];
            ValueInfo& s = V[c.inputs[0]];
            if (o.pl.valid && !s.pl.valid) try_place(m, (int)c.inputs[0], o.pl);
            continue;
        }
        if (c.kind != kCmdConcat) continue;
        ValueInfo& o = V[c.output];
        if (!o.pl.valid) new_root(m, (int)c.output, false);
        const Placement base = o.pl;
        const bool along_c = (o.rank == 4 && c.params[2] == 1) || (o.rank == 3 && c.params[2] == 2);
        int off = 0;
        for (size_t k = 0; k < c.inputs.size(); ++k) {
            const int in = (int)c.inputs[k];
            ValueInfo& x = V[in];
            Placement slice = base;
            if (along_c) {
                slice.offset += off;
                slice.slot = (base.slot >= 0 && off % 16 == 0) ? base.slot + off / 16 : -1;
                // a slice off the 16-channel grid: its producer cannot fold into
                // the root's slots, and a neighbour's group would miss it
                if (base.slot >= 0 && (off % 16 || x.C % 16)) m->roots[base.root].slots_complete = false;
            } else {
                slice.offset += int64_t(off) * x.W * base.cstride;
            }
            bool placed = false;
            const int pc = x.producer;
            if (pc >= 0 && e.commands[pc].kind == kCmdView && along_c) {
                const int src = (int)e.commands[pc].inputs[0];
                const ValueInfo& s = V[src];
                const int c0 = (int)(e.commands[pc].params[0] / (uint64_t(s.H) * s.W));
                const int start = off - c0;
                if (start >= 0 && start + s.C <= o.C && (base.slot < 0 || start % 16 == 0)) {
                    Placement ps = base;
                    ps.offset += start;
                    ps.slot = base.slot >= 0 ? base.slot + start / 16 : -1;
                    placed = try_place(m, src, ps);
                }
            } else if (pc >= 0 && e.commands[pc].kind == kCmdAlias) {
                // the reshape shares its source's memory; its own placement is
                // derived from the source in the forward pass
                placed = try_place(m, (int)e.commands[pc].inputs[0], slice);
            } else {
                placed = (!along_c || base.slot < 0 || off % 16 == 0) && try_place(m, in, slice);
            }
            if (!placed) copies.push_back(CopyJob{ci, in, slice});
            off += along_c ? x.C : x.H;
        }
    }
    place_sibling_convs(m);
    // forward: views / aliases / everything else
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        ValueInfo& o = V[c.output];
        if (c.kind == kCmdView) {
            const ValueInfo& s = V[c.inputs[0]];
            const int c0 = (int)(c.params[0] / (uint64_t(s.H) * s.W));
            if (!s.pl.valid) return fail(m, "view source without storage");
            o.pl = s.pl;
            o.pl.offset += c0;
            o.pl.slot = (s.pl.slot >= 0 && c0 % 16 == 0 && o.C % 16 == 0) ? s.pl.slot + c0 / 16 : -1;
            continue;
        }
        if (c.kind == kCmdAlias) {
            if (!V[c.inputs[0]].pl.valid) return fail(m, "alias source without storage");
            if (!o.pl.valid) o.pl = V[c.inputs[0]].pl;
            continue;
        }
        if (o.redirect >= 0) continue;  // fused conv output: never stored
        if (!o.pl.valid) new_root(m, (int)c.output, false);
    }
    // The network input arrives as fp32 NCHW.  When every consumer is a 3x3
    // pad-1 SiLU conv on at most 4 channels (the stem), those convs read it
    // directly (fp32 NCHW loader, channels zero-padded to 8); otherwise a
    // staging step writes an fp16 NHWC copy, channels zero-padded to 8.
    const uint32_t in_v = e.manifest.input_value;
    if (!V[in_v].consumers.empty()) {
        if (V[in_v].C % 8) V[in_v].cpad = (V[in_v].C + 7) / 8 * 8;
        bool direct = V[in_v].C <= 4 && V[in_v].rank == 4;
        for (int ci : V[in_v].consumers) {
            const EngineCommand& c = e.commands[ci];
            const AexrtConv2DDesc d = desc_of(c);
            direct = direct && c.kind == kCmdConvSilu && c.inputs[0] == in_v && d.kernel_h == 3 && d.kernel_w == 3 &&
                     d.pad_top == 1 && (d.stride_h == 1 || d.stride_h == 2) && !m->convs[ci].fused_residual &&
                     c.output != e.manifest.output_value;
        }
        m->input_nchw_direct = direct;
        m->input_needs_nhwc = !direct;
        if (!direct) new_root(m, (int)in_v, false);
    }
    return true;
}

// ---- weights ----------------------------------------------------------------------
bool constant_f32(AexrtYoloModel* m, uint32_t vid, std::vector<float>& out) {
    const EngineConstant& c = m->eng.constants[vid];
    if (!c.present) return false;
    out.resize(c.elements);
    if (c.precision == 2) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(c.raw.data());
        for (uint64_t i = 0; i < c.elements; ++i) {
            _Float16 v;
            std::memcpy(&v, &h[i], 2);
            out[i] = (float)v;
        }
    } else {
        std::memcpy(out.data(), c.raw.data(), c.elements * 4);
    }
    return true;
}

AexrtConv2DDesc desc_of(const EngineCommand& c) {
    AexrtConv2DDesc d;
    std::memcpy(&d, c.params.data(), sizeof(d));
    return d;
}

// Descriptor of a conv as launched: a zero-padded input (network input with
// C % 8 != 0) is convolved at its padded channel count.
AexrtConv2DDesc conv_desc_padded(AexrtYoloModel* m, size_t ci) {
    const EngineCommand& c = m->eng.commands[ci];
    AexrtConv2DDesc d = desc_of(c);
    const ValueInfo& x = m->vals[c.inputs[0]];
    if (x.cpad > x.C) d.in_channels = (uint32_t)x.cpad;
    return d;
}

// How an int8 conv quantizes its input (RT:23935-24318): an input of fewer
// than 4096 elements is quantized per (position, 4 channels) in the conv
// (RT:21478-21479, the dynamic kernel, pg16 or not); otherwise plan flag 16
// (engine.py:85-96) selects per-16-input-channel scales (RT:4770-4923), else
// one per-tensor scale.
void set_int8_mode(AexrtYoloModel* m, size_t ci) {
    ConvState& cs = m->convs[ci];
    const EngineCommand& c = m->eng.commands[ci];
    const AexrtConv2DDesc d = desc_of(c);
    const bool int8 = is_int8_algorithm(cs.algorithm);
    const uint64_t elems = uint64_t(d.batch) * d.in_channels * d.in_h * d.in_w;
    cs.dynamic = int8 && elems < kInt8PrequantMinElements;
    cs.pg16 = int8 && !cs.dynamic && (c.plan_flags & kPlanFlagInt8PerGroup) != 0;
}

uint32_t resolve_algorithm(AexrtYoloModel* m, size_t ci, uint32_t wanted) {
    const EngineCommand& c = m->eng.commands[ci];
    const AexrtConv2DDesc d = desc_of(c);
    const ValueInfo& x = m->vals[c.inputs[0]];
    // the raw network input is fp32 NCHW; an int8 or Winograd consumer gets
    // an fp16 NHWC copy of it (with amax slots), which needs C % 8 == 0
    const bool nhwc_input = !x.is_input || x.C % 8 == 0;
    if (is_int8_algorithm(wanted)) {
        const uint32_t kk = int8_kernel_elems(wanted);
        const bool family_ok = (wanted == 51) || (wanted == 52 && d.stride_h == 1) || (wanted == 53 && d.stride_h == 2);
        if (family_ok && can_use_int8(d, kk) && nhwc_input) return wanted;
        return 5;  // fail-closed fallback to the generic kernel
    }
    if (is_winograd_algorithm(wanted)) {
        // The reference plans Winograd F(2x2,3x3) for fp16 3x3 convs where its
        // autotuner measured it fastest.  On gfx950 the direct fp16 kernel
        // (halo-tile 3x3) beats the Winograd one on every such layer of the
        // network, so it runs them from the raw weights; the result is the same
        // conv within fp16 rounding.  aexrt_yolo_override_conv_algorithm(.., 40)
        // still selects the Winograd kernel.
        if (d.in_channels % 16 == 0 && d.out_channels % 8 == 0 && nhwc_input) return 5;
        if (winograd_shape_ok(d) && c.kind == kCmdConvSilu && nhwc_input) return wanted;
        return 5;
    }
    return wanted;
}

bool prepare_conv_weights(AexrtYoloModel* m, size_t ci) {
    const EngineCommand& c = m->eng.commands[ci];
    ConvState& cs = m->convs[ci];
    const AexrtConv2DDesc d = conv_desc_padded(m, ci);
    const uint32_t real_c = c.params[1];
    const uint32_t wid = c.inputs[1], bid = c.inputs[2];
    const EnginePacked& pk = m->eng.packed[wid];
    uint32_t layout = AEXRT_HIP_SRC_RAW_F32;
    const void* src = nullptr;
    uint64_t src_bytes = 0;
    const uint32_t a = cs.algorithm;
    const uint32_t kk = d.kernel_h * d.kernel_w;
    auto pk_ok = [&](uint32_t lay) {
        return pk.present && pk.layout == lay && pk.in_channels == d.in_channels && pk.out_channels == d.out_channels;
    };
    if (is_int8_algorithm(a) && pk_ok(8) && pk.elements == uint64_t(d.in_channels) * d.out_channels * kk) {
        layout = AEXRT_HIP_SRC_LAYOUT_INT8;
    } else if (is_winograd_algorithm(a) && pk_ok(3)) {
        layout = AEXRT_HIP_SRC_LAYOUT_WINO_F16;
    } else if (is_winograd_algorithm(a) && pk_ok(5)) {
        layout = AEXRT_HIP_SRC_LAYOUT_WINO_F32;
    } else if (!is_int8_algorithm(a) && !is_winograd_algorithm(a) && pk_ok(4) && kk == 1) {
        layout = AEXRT_HIP_SRC_LAYOUT_OC8_F16;
    } else if (!is_int8_algorithm(a) && !is_winograd_algorithm(a) && pk_ok(2) && kk == 9) {
        layout = AEXRT_HIP_SRC_LAYOUT_OC4_F16;
    }
    std::vector<float> padded;
    if (d.in_channels != real_c) {
        // zero-pad the input channels of the weight: [oc][real_c][kk] -> [oc][C][kk]
        std::vector<float> w;
        if (!constant_f32(m, wid, w) || w.size() != uint64_t(d.out_channels) * real_c * kk)
            return fail(m, "command " + std::to_string(ci) + ": conv weight is not a constant");
        padded.assign(uint64_t(d.out_channels) * d.in_channels * kk, 0.0f);
        for (uint32_t o = 0; o < d.out_channels; ++o)
            for (uint32_t ch = 0; ch < real_c; ++ch)
                for (uint32_t k = 0; k < kk; ++k)
                    padded[(uint64_t(o) * d.in_channels + ch) * kk + k] = w[(uint64_t(o) * real_c + ch) * kk + k];
        layout = AEXRT_HIP_SRC_RAW_F32;
        src = padded.data();
        src_bytes = padded.size() * 4;
    } else if (layout != AEXRT_HIP_SRC_RAW_F32) {
        src = pk.data.data();
        src_bytes = pk.data.size();
    } else {
        const EngineConstant& wc = m->eng.constants[wid];
        if (!wc.present) return fail(m, "command " + std::to_string(ci) + ": conv weight is not a constant");
        layout = wc.precision == 2 ? AEXRT_HIP_SRC_RAW_F16 : AEXRT_HIP_SRC_RAW_F32;
        src = wc.raw.data();
        src_bytes = wc.raw.size();
    }
    const WeightGeom g = weight_geom(d, a);
    std::vector<uint8_t> host(g.nbytes);
    std::vector<float> scale(d.out_channels, 0.0f);
    if (!aexrt_hip_pack_conv_weight(&d, a, layout, src, src_bytes, host.data(), host.size(),
                                    is_int8_algorithm(a) ? scale.data() : nullptr))
        return fail(m, "command " + std::to_string(ci) + ": " + last_error());
    std::vector<float> bias;
    if (!constant_f32(m, bid, bias) || bias.size() != d.out_channels)
        return fail(m, "command " + std::to_string(ci) + ": conv bias is not a constant of out_channels values");
    cs.w = dev_alloc(m, host.size());
    cs.w_bytes = host.size();
    cs.bias = static_cast<float*>(dev_alloc(m, bias.size() * 4));
    if (!cs.w || !cs.bias) return fail(m, "out of device memory for weights");
    if (!check_hip(hipMemcpy(cs.w, host.data(), host.size(), hipMemcpyHostToDevice), "weight upload") ||
        !check_hip(hipMemcpy(cs.bias, bias.data(), bias.size() * 4, hipMemcpyHostToDevice), "bias upload"))
        return fail(m, last_error());
    cs.scale = nullptr;
    if (is_int8_algorithm(a)) {
        cs.scale = static_cast<float*>(dev_alloc(m, scale.size() * 4));
        if (!cs.scale || !check_hip(hipMemcpy(cs.scale, scale.data(), scale.size() * 4, hipMemcpyHostToDevice),
                                    "scale upload"))
            return fail(m, "weight scale upload failed");
    }
    return true;
}

// Weights and bias of a sibling pair (ci first): the packed rows of both
// convs ([OCp][Kp], OCp = OC here) back to back, as one conv's would be.
bool pair_conv_weights(AexrtYoloModel* m, size_t ci) {
    ConvState& a = m->convs[ci];
    const ConvState& b = m->convs[m->sibling[ci]];
    const uint32_t ca = desc_of(m->eng.commands[ci]).out_channels;
    const uint32_t cb = desc_of(m->eng.commands[m->sibling[ci]]).out_channels;
    auto direct = [](uint32_t k) { return !is_int8_algorithm(k) && !is_winograd_algorithm(k); };
    if (!direct(a.algorithm) || !direct(b.algorithm) || a.w_bytes % ca || b.w_bytes % cb || a.w_bytes / ca != b.w_bytes / cb)
        return true;  // launched one by one
    a.w_pair = dev_alloc(m, a.w_bytes + b.w_bytes);
    a.bias_pair = static_cast<float*>(dev_alloc(m, (ca + cb) * 4u));
    if (!a.w_pair || !a.bias_pair) return fail(m, "out of device memory for weights");
    uint8_t* w = static_cast<uint8_t*>(a.w_pair);
    if (!check_hip(hipMemcpy(w, a.w, a.w_bytes, hipMemcpyDeviceToDevice), "pair weights") ||
        !check_hip(hipMemcpy(w + a.w_bytes, b.w, b.w_bytes, hipMemcpyDeviceToDevice), "pair weights") ||
        !check_hip(hipMemcpy(a.bias_pair, a.bias, ca * 4u, hipMemcpyDeviceToDevice), "pair bias") ||
        !check_hip(hipMemcpy(a.bias_pair + ca, b.bias, cb * 4u, hipMemcpyDeviceToDevice), "pair bias"))
        return fail(m, last_error());
    a.pair_src[0] = a.w;
    a.pair_src[1] = b.w;
    return true;
}

// ---- launch list ------------------------------------------------------------------
AexrtHipTensorView view_of(AexrtYoloModel* m, int v) {
    const ValueInfo& x = m->vals[v];
    const Root& r = m->roots[x.pl.root];
    AexrtHipTensorView tv{};
    tv.data = m->arena + r.byte_offset + x.pl.offset * (r.f32 ? 4 : 2);
    tv.n_stride = x.pl.nstride;
    tv.c_stride = x.pl.cstride;
    tv.amax_slots = x.pl.slot >= 0 && r.slots_read ? m->slots + x.pl.slot : nullptr;
    tv.amax_stripes = tv.amax_slots ? kSlotStripes : 0u;
    tv.amax_stripe_stride = m->slot_stride;
    return tv;
}

AexrtHipTensorView view_of_pl(AexrtYoloModel* m, const Placement& pl) {
    const Root& r = m->roots[pl.root];
    AexrtHipTensorView tv{};
    tv.data = m->arena + r.byte_offset + pl.offset * (r.f32 ? 4 : 2);
    tv.n_stride = pl.nstride;
    tv.c_stride = pl.cstride;
    tv.amax_slots = pl.slot >= 0 && r.slots_read ? m->slots + pl.slot : nullptr;
    tv.amax_stripes = tv.amax_slots ? kSlotStripes : 0u;
    tv.amax_stripe_stride = m->slot_stride;
    return tv;
}

bool is_f32(AexrtYoloModel* m, int v) { return m->roots[m->vals[v].pl.root].f32; }

std::string conv_label(const EngineCommand& c, size_t ci, uint32_t alg) {
    char buf[192];
    std::snprintf(buf, sizeof(buf), "cmd#%zu %s %ux%ux%u -> %ux%ux%u k%u s%u alg=%s", ci, kind_name(c.kind), c.params[1],
                  c.params[2], c.params[3], c.params[4], c.params[5], c.params[6], c.params[7], c.params[9],
                  algorithm_name(alg));
    return buf;
}

// ---- plan-time kernel choice ---------------------------------------------------
// The reference's kernel plan records, per conv, the kernel its autotuner
// measured fastest on the reference's GPU.  Here every conv gets the
// implicit-GEMM or halo tile measured fastest on this one: each candidate runs
// once to warm up, then kTuneReps times between two events on the model stream,
// on the conv's own buffers (the first real run overwrites what they leave,
// and clears the amax slots at its start).  Convs of one shape share the
// result.  AEXRT_HIP_AUTOTUNE=0 keeps the heuristic choice.
constexpr int kTuneReps = 4;

std::string tune_key(const ConvParams& p, bool int8) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), "%d|%d|%d|%d,%d,%d,%d|%d,%d,%d,%d,%d|%d,%d|%lld,%d,%lld,%d|%d,%d|%u", int8 ? 1 : 0,
                  p.flags, p.loader, p.N, p.H, p.W, p.C, p.OC, p.KH, p.KW, p.S, p.P, p.OH, p.OW,
                  (long long)p.x_nstride, p.x_cstride, (long long)p.y_nstride, p.y_cstride, p.res ? 1 : 0,
                  p.acc_out ? 1 : 0, p.x_slots.stripes);
    std::string k = buf;
    if (p.fuse_1x1) {
        // the fused 1x1: its output channels, flags and output view
        std::snprintf(buf, sizeof(buf), "|f%d,%d,%lld,%d", p.fuse_1x1->OC, p.fuse_1x1->flags,
                      (long long)p.fuse_1x1->y_nstride, p.fuse_1x1->y_cstride);
        k += buf;
    }
    if (p.yup) {
        // the upsample copy: its view
        std::snprintf(buf, sizeof(buf), "|u%lld,%d", (long long)p.yup_nstride, p.yup_cstride);
        k += buf;
    }
    if (p.xup) {
        // the upsampled input source: its channels and view
        std::snprintf(buf, sizeof(buf), "|x%d,%d,%lld,%d", p.xup_c0, p.xup_cn, (long long)p.xup_nstride,
                      p.xup_cstride);
        k += buf;
    }
    return k;
}

bool same_choice(const ConvChoice& a, const ConvChoice& b) {
    return a.kind == b.kind && a.jn == b.jn && a.pw == b.pw && a.ksw == b.ksw && a.tr == b.tr && a.tc == b.tc &&
           a.cc == b.cc && a.nw == b.nw;
}

// AEXRT_HIP_TUNE_CACHE=<file>: measured choices are read from the file at load
// (each still checked against the shape's candidates) and the file is
// rewritten with every choice of the model, so that later loads of the same
// engine (or of another with the same conv shapes) launch the same kernels.
// One line per conv shape: key, tab, kind jn pw ksw tr tc cc nw; a measured
// schedule in the same form; a list-scheduled network's lanes as
// "lanes <input dims> commands <n>", tab, one digit per step.
void load_tune_cache(AexrtYoloModel* m) {
    std::ifstream f(m->tune_cache);
    std::string line;
    while (std::getline(f, line)) {
        const size_t tab = line.find('\t');
        if (tab == std::string::npos) continue;
        if (line.compare(0, 6, "lanes ") == 0) {
            const std::string plan = line.substr(tab + 1);
            if (!plan.empty() && plan.find_first_not_of("0123") == std::string::npos)
                m->lane_plans[line.substr(0, tab)] = plan;
            continue;
        }
        ConvChoice c{};
        if (std::sscanf(line.c_str() + tab + 1, "%d %d %d %d %d %d %d %d", &c.kind, &c.jn, &c.pw, &c.ksw, &c.tr,
                        &c.tc, &c.cc, &c.nw) != 8)
            continue;
        if (line.compare(0, 4, "cmd ") == 0 || line.compare(0, 10, "chain cmd ") == 0)
            m->refined[line.substr(0, tab)] = c;  // a conv's (or a chain's tile) choice measured in the network
        else if (line.compare(0, 9, "schedule ") == 0)
            m->schedules[line.substr(0, tab)] =
                Schedule{c.kind, c.jn, c.pw, (uint32_t)c.ksw, (uint32_t)c.tr, (uint32_t)c.tc,
                         c.cc & 3};  // merge, lanes, fusion, pairs, branches, paired branches, superblocks
        else
            m->tuned[line.substr(0, tab)] = c;
    }
}

void save_tune_cache(AexrtYoloModel* m) {
    const std::string tmp = m->tune_cache + ".tmp";
    {
        std::ofstream f(tmp, std::ios::trunc);
        auto put = [&](const std::string& key, const ConvChoice& c) {
            f << key << '\t' << c.kind << ' ' << c.jn << ' ' << c.pw << ' ' << c.ksw << ' ' << c.tr << ' ' << c.tc
              << ' ' << c.cc << ' ' << c.nw << '\n';
        };
        for (const auto& [key, c] : m->tuned) put(key, c);
        for (const auto& [key, c] : m->refined) put(key, c);
        for (const auto& [key, v] : m->schedules)
            put(key, ConvChoice{v.first, v.second, v.fuse, (int)v.mask, (int)v.chains, (int)v.dual, v.super, 0});
        for (const auto& [key, plan] : m->lane_plans) f << key << '\t' << plan << '\n';
        if (!f) return;
    }
    std::rename(tmp.c_str(), m->tune_cache.c_str());
}

// Candidates of a shape kept for the measurement in the running network.
constexpr int kContextCands = 4;

bool tune_conv(AexrtYoloModel* m, ConvParams& p, bool int8, std::vector<ConvChoice>* top) {
    const std::string key = tune_key(p, int8);
    std::vector<ConvChoice> cand(kMaxConvChoices);
    const int n = enumerate_conv_choices(p, int8, cand.data(), kMaxConvChoices);
    if (n >= kMaxConvChoices)
        std::fprintf(stderr, "aexrt tune %s: %d candidates, the enumeration cap; the rest are not measured\n",
                     key.c_str(), n);
    auto it = m->tuned.find(key);
    if (it != m->tuned.end()) {
        for (int i = 0; i < n; ++i)
            if (same_choice(cand[i], it->second)) {
                p.choice = it->second;
                auto tt = m->tuned_top.find(key);
                if (top) *top = tt != m->tuned_top.end() ? tt->second : std::vector<ConvChoice>{it->second};
                return true;
            }
        m->tuned.erase(it);  // a cached choice this build does not offer
    }
    std::vector<std::pair<float, ConvChoice>> timed;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!check_hip(hipEventCreate(&e0), "tune event") || !check_hip(hipEventCreate(&e1), "tune event")) {
        if (e0) (void)hipEventDestroy(e0);
        return fail(m, last_error());
    }
    ConvChoice best{};
    float best_ms = 0.0f;
    bool ok = true;
    for (int i = 0; i < n && ok; ++i) {
        ConvParams q = p;
        q.choice = cand[i];
        if (launch_conv_igemm(q, int8, m->stream) != hipSuccess) continue;  // rejected on the host
        ok = check_hip(hipEventRecord(e0, m->stream), "tune record");
        for (int r = 0; r < kTuneReps && ok; ++r) ok = check_hip(launch_conv_igemm(q, int8, m->stream), "tune launch");
        ok = ok && check_hip(hipEventRecord(e1, m->stream), "tune record") &&
             check_hip(hipEventSynchronize(e1), "tune sync");
        float ms = 0.0f;
        ok = ok && check_hip(hipEventElapsedTime(&ms, e0, e1), "tune elapsed");
        if (ok) timed.emplace_back(ms, cand[i]);
        if (ok && (best.kind == 0 || ms < best_ms)) {
            best = cand[i];
            best_ms = ms;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!ok) return fail(m, last_error());
    std::stable_sort(timed.begin(), timed.end(),
                     [](const std::pair<float, ConvChoice>& a, const std::pair<float, ConvChoice>& b) {
                         return a.first < b.first;
                     });
    std::vector<ConvChoice> fastest;
    for (size_t i = 0; i < timed.size() && (int)fastest.size() < kContextCands; ++i) fastest.push_back(timed[i].second);
    m->tuned[key] = best;
    m->tuned_top[key] = fastest;
    if (top) *top = fastest;
    p.choice = best;
    if (m->tune_log)
        std::fprintf(stderr, "aexrt tune %s: kind %d jn %d pw %d ksw %d tr %d tc %d cc %d nw %d  %.2f us (%d candidates)\n",
                     key.c_str(), best.kind, best.jn, best.pw, best.ksw, best.tr, best.tc, best.cc, best.nw,
                     best_ms * 1000.0f / kTuneReps, n);
    return true;
}

// ---- multi-stream schedule ---------------------------------------------------------
// Every value lives in its own region of a root (concat inputs in disjoint channel
// slices of the concat's root) and is written once per run, so the only ordering a
// step needs is after the earlier steps that write a root it reads (read after
// write), and everything after the slot clear.  Two producers of slices of one root
// touch disjoint bytes and disjoint amax slot groups, so they may run concurrently.
// Lanes, by the dependency rule: a step continues the lane of its latest
// dependency when that lane has not moved on, else takes an idle lane (else the
// least recently used one, which then orders it after that lane's last step
// too); dependencies on other lanes become event waits.  The captured graph thus
// has parallel branches (the head's box and class chains, the finest head level
// beside the rest of the neck).  The rule looks at step order only: a head branch
// whose input was produced early can land behind the rest of the neck.  List
// scheduling instead takes the steps' times measured in the network on one lane
// and puts each step on the lane where it can start first (after its
// dependencies' estimated ends and its lane's last step), preferring a lane that
// ends with one of its dependencies (no cross-lane wait).  Which of the two runs
// faster is measured at load.
// Whether step i must follow the earlier step j: it reads a root j writes,
// either one touches every root, or both meet in a grid barrier.
bool step_depends(const Step& i, const Step& j) {
    bool dep = i.all || j.all || (i.grid_sync && j.grid_sync);
    for (int r : i.reads)
        for (int w : j.writes) dep = dep || r == w;
    return dep;
}

void schedule_steps(AexrtYoloModel* m) {
    auto& st = m->steps;
    const int nl = std::max(1, std::min(kLanes, m->n_lanes));
    const int n = (int)st.size();
    for (int i = 0; i < n; ++i) {
        st[i].deps.clear();
        st[i].signal = false;
        for (int j = i - 1; j >= 0; --j)
            if (step_depends(st[i], st[j])) st[i].deps.push_back(j);
    }
    int last[kLanes];
    for (int l = 0; l < kLanes; ++l) last[l] = -1;
    const bool planned = m->lane_policy == 2 && (int)m->lane_plan.size() == n;
    const bool listed = m->lane_policy == 1 && (int)m->step_ms.size() == n;
    std::vector<double> end(n, 0.0);  // list scheduling: estimated end of each step
    double lane_end[kLanes] = {};
    for (int i = 0; i < n; ++i) {
        int lane = -1;
        if (nl == 1) {
            lane = 0;
        } else if (planned) {
            lane = std::min(nl - 1, std::max(0, m->lane_plan[i] - '0'));
        } else if (listed) {
            double ready = 0.0;
            for (int d : st[i].deps) ready = std::max(ready, end[d]);
            double best = 0.0;
            bool best_follows = false;
            constexpr double kTie = 1e-4;  // ms: starts this close count as equal
            for (int l = 0; l < nl; ++l) {
                const double start = std::max(ready, lane_end[l]);
                bool follows = false;
                for (int d : st[i].deps) follows = follows || last[l] == d;
                if (lane < 0 || start < best - kTie || (start <= best + kTie && follows && !best_follows)) {
                    lane = l;
                    best = start;
                    best_follows = follows;
                }
            }
            end[i] = best + std::max(0.0f, m->step_ms[i]);
            lane_end[lane] = end[i];
        } else {
            int best = -1;
            for (int l = 0; l < nl; ++l)
                for (int d : st[i].deps)
                    if (last[l] == d && d > best) {
                        best = d;
                        lane = l;
                    }
            if (lane < 0) {
                for (int l = 0; l < nl && lane < 0; ++l)
                    if (last[l] < 0) lane = l;
                if (lane < 0) {
                    lane = 0;
                    for (int l = 1; l < nl; ++l)
                        if (last[l] < last[lane]) lane = l;
                }
            }
        }
        st[i].lane = lane;
        for (int d : st[i].deps)
            if (st[d].lane != lane) st[d].signal = true;
        last[lane] = i;
    }
}

// The lanes of the current schedule, one digit per step.
std::string lane_digits(const AexrtYoloModel* m) {
    std::string s;
    for (const Step& x : m->steps) s += (char)('0' + x.lane);
    return s;
}

// Key of a conv's choice measured in the network: the command, its algorithm
// and its shape.  Overriding a conv's algorithm and restoring it finds the
// first measurement again, so the restored model runs the same kernels.
std::string refined_key(size_t ci, uint32_t alg, const ConvParams& p, bool int8) {
    return "cmd " + std::to_string(ci) + " alg " + std::to_string(alg) + " " + tune_key(p, int8);
}

// Without measurement (AEXRT_HIP_AUTOTUNE=0) a conv still takes a cached
// choice when the tune cache has one this build offers: its choice measured in
// the network first, else its shape's isolated measurement; otherwise the
// heuristics (choice kind 0).
void apply_cached_choice(AexrtYoloModel* m, size_t ci, uint32_t alg, ConvParams& p, bool int8) {
    std::vector<ConvChoice> all(kMaxConvChoices);
    const int na = enumerate_conv_choices(p, int8, all.data(), kMaxConvChoices);
    // a fused 1x1 runs on the 32x32-MFMA kernel only, an upsample copy or an
    // upsampled input source on the streaming 1x1 kernel: without a measured
    // choice, the first tile that fits
    if ((p.fuse_1x1 || p.yup || p.xup) && na > 0) p.choice = all[0];
    if (m->tune_cache.empty()) return;
    auto offered = [&](const ConvChoice& c) {
        for (int k = 0; k < na; ++k)
            if (same_choice(all[k], c)) return true;
        return false;
    };
    auto rf = m->refined.find(refined_key(ci, alg, p, int8));
    if (rf != m->refined.end() && offered(rf->second)) {
        p.choice = rf->second;
        return;
    }
    auto tu = m->tuned.find(tune_key(p, int8));
    if (tu != m->tuned.end() && offered(tu->second)) {
        p.choice = tu->second;
        return;
    }
    if (p.yup || p.xup) {
        // the same conv measured without the upsample copy or source: its
        // tile, when those kernel instances include it
        ConvParams q = p;
        q.yup = nullptr;
        q.xup = nullptr;
        auto rq = m->refined.find(refined_key(ci, alg, q, int8));
        if (rq != m->refined.end() && offered(rq->second)) {
            p.choice = rq->second;
            return;
        }
        auto tq = m->tuned.find(tune_key(q, int8));
        if (tq != m->tuned.end() && offered(tq->second)) p.choice = tq->second;
    }
}

// Labels of the conv steps name the kernel and tile that runs (it changes as
// the tile choices are measured): "<command> alg=<plan family> kernel=<kernel>".
void label_steps(AexrtYoloModel* m) {
    for (Step& st : m->steps)
        if (st.family) st.label = st.head + " kernel=" + st.family() + st.tail;
}

// Kernel parameters of the head branch led by 3x3 conv ci (its a, b, c);
// false when the three convs do not fit the chain kernel.
bool chain_params_of(AexrtYoloModel* m, size_t ci, ConvParams (&br)[3]) {
    const Engine& e = m->eng;
    const ConvState& cs = m->convs[ci];
    const int ib = cs.chain_b, ic = cs.chain_c;
    const ConvState& bs = m->convs[ib];
    const ConvState& ccs = m->convs[ic];
    const AexrtHipTensorView xv = view_of(m, (int)e.commands[ci].inputs[0]);
    const AexrtHipTensorView t1 = view_of(m, cs.out_value), t2 = view_of(m, bs.out_value);
    const AexrtHipTensorView yv = view_of(m, ccs.out_value);
    const uint32_t flags_c = (e.commands[ic].kind == kCmdConvSilu ? AEXRT_HIP_CONV_SILU : 0u) |
                             (is_f32(m, ccs.out_value) ? AEXRT_HIP_CONV_OUT_F32 : 0u);
    std::string why;
    int tr = 0, tc = 0;
    return !is_f32(m, cs.out_value) && !is_f32(m, bs.out_value) &&
           build_conv_params(conv_desc_padded(m, ci), cs.algorithm, AEXRT_HIP_CONV_SILU, xv, cs.w, nullptr, cs.bias,
                             nullptr, t1, nullptr, br[0], why) &&
           build_conv_params(conv_desc_padded(m, (size_t)ib), bs.algorithm, AEXRT_HIP_CONV_SILU, t1, bs.w, nullptr,
                             bs.bias, nullptr, t2, nullptr, br[1], why) &&
           build_conv_params(conv_desc_padded(m, (size_t)ic), ccs.algorithm, flags_c, t2, ccs.w, nullptr, ccs.bias,
                             nullptr, yv, nullptr, br[2], why) &&
           !chain_shape_error(br[0], br[1], br[2]) && chain_tile(br[0], br[1], br[2], tr, tc);
}

// Undoes the head branch led by ci (its convs then run on their own).
void unchain(AexrtYoloModel* m, size_t ci) {
    const Engine& e = m->eng;
    ConvState& cs = m->convs[ci];
    m->vals[e.commands[ci].output].elided = false;
    m->vals[e.commands[cs.chain_b].output].elided = m->convs[cs.chain_b].fused_1x1 >= 0;
    cs.chain_b = cs.chain_c = -1;
}

// The step of the head branch led by 3x3 conv ci (3x3 chain_b, 1x1
// chain_c), with the branch of another 3x3 conv over the same input in the
// same launch when there is one (the level's box and class branches);
// built = false (and the branch undone) when it does not fit the kernel.
bool build_chain_step(AexrtYoloModel* m, size_t ci, std::vector<bool>& done, bool& built) {
    built = false;
    const Engine& e = m->eng;
    auto& V = m->vals;
    ConvState& cs = m->convs[ci];
    ConvParams br0[3];
    if (!chain_params_of(m, ci, br0)) {
        unchain(m, ci);
        return true;
    }
    auto dual = [&](size_t c) {
        for (size_t k = 0; k < m->chains.size() && k < 32; ++k)
            if (m->chains[k][0] == (int)c) return ((m->chain_dual >> k) & 1u) != 0;
        return false;
    };
    int partner = -1;
    ConvParams br1[3];
    for (size_t cj = ci + 1; cj < e.commands.size() && partner < 0 && dual(ci); ++cj) {
        if (done[cj] || m->convs[cj].chain_b < 0 || e.commands[cj].inputs[0] != e.commands[ci].inputs[0] || !dual(cj))
            continue;
        if (!chain_params_of(m, cj, br1)) continue;
        LaunchProbe probe{};
        set_launch_probe(&probe);
        const hipError_t pe = launch_conv_chain2(br0, br1, 0, 0, nullptr);
        set_launch_probe(nullptr);
        if (pe == hipSuccess) partner = (int)cj;
    }
    const int ib = cs.chain_b, ic = cs.chain_c;
    std::string tail = " then cmd#" + std::to_string(e.src_cmd[ib]) + " then 1x1 cmd#" + std::to_string(e.src_cmd[ic]);
    std::vector<int> writes = {V[m->convs[ic].out_value].pl.root};
    // the launch's tile: measured before (this load or the tune cache) when the
    // kernel still offers it, else the largest that fits until measured
    AexrtYoloModel::ChainStep rec;
    rec.ci = ci;
    rec.partner = partner;
    rec.step = m->steps.size();
    rec.key = "chain cmd " + std::to_string(ci) + " " + std::to_string(br0[0].N) + "x" + std::to_string(br0[0].C) +
              "x" + std::to_string(br0[0].H) + "x" + std::to_string(br0[0].W) + (partner >= 0 ? " two" : " one");
    cs.chain_tr = cs.chain_tc = 0;
    auto rf = m->refined.find(rec.key);
    if (rf != m->refined.end()) {
        int tr[16], tc[16];
        const int n = enumerate_chain_tiles(br0, partner >= 0 ? br1 : nullptr, tr, tc, 16);
        for (int k = 0; k < n && !rec.done; ++k)
            if (tr[k] == rf->second.tr && tc[k] == rf->second.tc) {
                cs.chain_tr = tr[k];
                cs.chain_tc = tc[k];
                rec.done = true;
            }
    }
    m->chain_steps.push_back(rec);
    // the launch reads the tile when it runs, so a tile measured later applies
    // (m->convs is sized once at load: the pointer stays valid)
    const ConvState* tile = &cs;
    if (partner >= 0) {
        const ConvState& ps = m->convs[partner];
        const std::array<ConvParams, 3> a0{br0[0], br0[1], br0[2]}, a1{br1[0], br1[1], br1[2]};
        m->steps.push_back(Step{(int)ci, "", [a0, a1, tile](hipStream_t s) {
                                    return launch_conv_chain2(a0.data(), a1.data(), tile->chain_tr, tile->chain_tc, s);
                                }});
        m->steps.back().family = [a0, a1, tile] {
            LaunchProbe probe{};
            set_launch_probe(&probe);
            (void)launch_conv_chain2(a0.data(), a1.data(), tile->chain_tr, tile->chain_tc, nullptr);
            set_launch_probe(nullptr);
            return std::string(probe.name);
        };
        tail += " + cmd#" + std::to_string(e.src_cmd[partner]) + " then cmd#" + std::to_string(e.src_cmd[ps.chain_b]) +
                " then 1x1 cmd#" + std::to_string(e.src_cmd[ps.chain_c]);
        writes.push_back(V[m->convs[ps.chain_c].out_value].pl.root);
        done[partner] = done[ps.chain_b] = done[ps.chain_c] = true;
    } else {
        const std::array<ConvParams, 3> a0{br0[0], br0[1], br0[2]};
        m->steps.push_back(Step{(int)ci, "", [a0, tile](hipStream_t s) {
                                    return launch_conv_chain(a0[0], a0[1], a0[2], tile->chain_tr, tile->chain_tc, s);
                                }});
        m->steps.back().family = [a0, tile] {
            LaunchProbe probe{};
            set_launch_probe(&probe);
            (void)launch_conv_chain(a0[0], a0[1], a0[2], tile->chain_tr, tile->chain_tc, nullptr);
            set_launch_probe(nullptr);
            return std::string(probe.name);
        };
    }
    Step& st = m->steps.back();
    st.head = conv_label(e.commands[ci], e.src_cmd[ci], cs.algorithm);
    st.tail = tail;
    st.reads = {V[e.commands[ci].inputs[0]].pl.root};
    st.writes = writes;
    done[ib] = done[ic] = true;
    built = true;
    return true;
}

// The superblock step of bottleneck pair (ci, its pair_b): both 3x3 convs in
// one launch (conv_pair.h); built = false (and the pair undone: both convs
// then run on their own) when the launcher refuses it, e.g. an int8 grid
// that the GPU cannot hold at once.
bool build_pair_step(AexrtYoloModel* m, size_t ci, int k, std::vector<bool>& done, bool& built) {
    built = false;
    const Engine& e = m->eng;
    auto& V = m->vals;
    ConvState& cs = m->convs[ci];
    const int cj = cs.pair_b;
    ConvState& bs = m->convs[cj];
    const bool int8 = is_int8_algorithm(cs.algorithm);
    auto undo = [&] {
        V[e.commands[ci].output].elided = false;
        bs.pair_a = -1;
        cs.pair_b = -1;
        return true;
    };
    const int xv = (int)e.commands[ci].inputs[0], tv = (int)e.commands[ci].output;
    AexrtHipTensorView xvw = view_of(m, xv), tvw = view_of(m, tv), yvw = view_of(m, bs.out_value);
    if (int8 && !tvw.amax_slots) tvw.amax_slots = xvw.amax_slots;  // read only through the barrier's amax words
    const uint32_t fa = AEXRT_HIP_CONV_SILU, fb = AEXRT_HIP_CONV_SILU | (bs.fused_residual ? AEXRT_HIP_CONV_RESIDUAL : 0u);
    ConvParams pa{}, pb{};
    std::string why;
    if (!build_conv_params(conv_desc_padded(m, ci), cs.algorithm, fa, xvw, cs.w, cs.scale, cs.bias, nullptr, tvw,
                           nullptr, pa, why) ||
        !build_conv_params(conv_desc_padded(m, (size_t)cj), bs.algorithm, fb, tvw, bs.w, bs.scale, bs.bias,
                           bs.fused_residual ? &xvw : nullptr, yvw, nullptr, pb, why))
        return undo();
    uint32_t* sync = int8 ? m->pair_sync + (size_t)k * kPairSyncWordsHost : nullptr;
    uint32_t* err = int8 ? m->pair_err : nullptr;
    {
        LaunchProbe probe{};
        set_launch_probe(&probe);
        const hipError_t pe = launch_conv_pair(pa, pb, int8, 0, sync, err, nullptr, nullptr, nullptr);
        set_launch_probe(nullptr);
        if (pe != hipSuccess) return undo();
    }
    m->steps.push_back(Step{(int)ci, "", [pa, pb, int8, sync, err](hipStream_t s) {
                                return launch_conv_pair(pa, pb, int8, 0, sync, err, nullptr, nullptr, s);
                            }});
    Step& st = m->steps.back();
    st.family = [pa, pb, int8, sync, err] {
        LaunchProbe probe{};
        set_launch_probe(&probe);
        (void)launch_conv_pair(pa, pb, int8, 0, sync, err, nullptr, nullptr, nullptr);
        set_launch_probe(nullptr);
        return std::string(probe.name);
    };
    st.head = conv_label(e.commands[ci], e.src_cmd[ci], cs.algorithm);
    st.tail = " then cmd#" + std::to_string(e.src_cmd[cj]) + " (C2f bottleneck superblock)";
    st.reads = {V[xv].pl.root};
    st.writes = {V[bs.out_value].pl.root};
    st.grid_sync = int8;
    done[cj] = true;
    built = true;
    return true;
}

void set_upsampled_input(AexrtYoloModel* m, ConvParams& p, int ci);

// The int8 1x1 conv that reads nearest 2x resize ci's output, a 16-channel
// aligned slice of a concat root, as its only reader (the concat over the
// whole root read by that conv alone, placed without a copy): -1 when there
// is none or the streaming kernel does not take the conv with the source.
int upsample_reader(AexrtYoloModel* m, size_t ci) {
    const Engine& e = m->eng;
    const EngineCommand& c = e.commands[ci];
    const int src = (int)c.inputs[0], o = (int)c.output;
    const ValueInfo& ov = m->vals[o];
    if (!ov.pl.valid || ov.C % 16 || ov.pl.offset % 16) return -1;
    for (int u : ov.consumers)
        if (e.commands[u].kind != kCmdConcat) return -1;
    for (const CopyJob& j : m->copies)
        if (j.src == o) return -1;
    const int R = ov.pl.root;
    int cat = -1;
    for (size_t v = 0; v < m->vals.size(); ++v) {
        const ValueInfo& x = m->vals[v];
        if (x.pl.valid && x.pl.root == R && x.pl.offset == 0 && x.C == m->roots[R].C && (int)v != o) cat = (int)v;
    }
    if (cat < 0 || m->vals[cat].consumers.size() != 1) return -1;
    const int k = m->vals[cat].consumers[0];
    const ConvState& ks = m->convs[k];
    if (!ks.is_conv || (int)e.commands[k].inputs[0] != cat || !is_int8_algorithm(ks.algorithm) || ks.pg16 ||
        ks.dynamic || ks.fused_residual || !m->roots[R].slots_complete || m->up_read[k] >= 0)
        return -1;
    const AexrtConv2DDesc d = desc_of(e.commands[k]);
    if (d.kernel_h != 1 || d.kernel_w != 1 || is_f32(m, ks.out_value)) return -1;
    const AexrtHipTensorView xv = view_of(m, cat), sv = view_of(m, src), yv = view_of(m, ks.out_value);
    if (!xv.amax_slots || !sv.amax_slots) return -1;
    // the kernel reads both views through one resource: within 4 GB of each other
    const uintptr_t xa = reinterpret_cast<uintptr_t>(xv.data), sa = reinterpret_cast<uintptr_t>(sv.data);
    const ValueInfo& cv = m->vals[cat];
    const ValueInfo& srcv = m->vals[src];
    const uintptr_t xe = xa + (uintptr_t)(cv.N * xv.n_stride) * 2, se = sa + (uintptr_t)(srcv.N * sv.n_stride) * 2;
    if (std::max(xe, se) - std::min(xa, sa) > 0xFFFFFFF0ull) return -1;
    ConvParams p{};
    std::string why;
    const uint32_t flags = e.commands[k].kind == kCmdConvSilu ? AEXRT_HIP_CONV_SILU : 0u;
    if (!build_conv_params(conv_desc_padded(m, (size_t)k), ks.algorithm, flags, xv, ks.w, ks.scale, ks.bias, nullptr,
                           yv, nullptr, p, why))
        return -1;
    set_upsampled_input(m, p, (int)ci);
    ConvChoice probe[4];
    return enumerate_conv_choices(p, true, probe, 4) > 0 ? k : -1;
}

// Nearest 2x resizes that never launch (AEXRT_HIP_FOLD_UPSAMPLE=0: every
// resize launches; =copy: the producer form only).  Where the one reader of
// the resize's output is an int8 1x1 conv over its concat, that conv reads
// the resize's input at half resolution instead (ConvParams::xup): the
// upsample is never stored.  Otherwise, where the resize's input comes from
// an int8 1x1 conv, that conv writes the upsample too (ConvParams::yup), so
// the resize neither launches nor reads the conv output again.  Candidates
// here; a producer whose shape and views the kernel does not take keeps its
// resize (build_steps).
void setup_upsample_folds(AexrtYoloModel* m) {
    const Engine& e = m->eng;
    m->up_fold.assign(e.commands.size(), -1);
    m->up_read.assign(e.commands.size(), -1);
    const char* env = std::getenv("AEXRT_HIP_FOLD_UPSAMPLE");
    if (env && env[0] == '0') return;
    const bool reader_form = !(env && std::strcmp(env, "copy") == 0);
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        if (c.kind != kCmdResize || c.inputs.empty()) continue;
        const ValueInfo& x = m->vals[c.inputs[0]];
        const ValueInfo& o = m->vals[c.output];
        if (o.N != x.N || o.C != x.C || o.H != 2 * x.H || o.W != 2 * x.W || is_f32(m, c.output)) continue;
        if (reader_form) {
            const int k = upsample_reader(m, ci);
            if (k >= 0) {
                m->up_read[k] = (int)ci;
                m->up_read[ci] = k;
                continue;
            }
        }
        if (x.producer < 0) continue;
        const int pc = x.producer;
        const ConvState& cs = m->convs[pc];
        if (!cs.is_conv || cs.out_value != (int)c.inputs[0] || !is_int8_algorithm(cs.algorithm) || cs.pg16 ||
            cs.dynamic || cs.fused_residual || cs.pair_a >= 0 || cs.pair_b >= 0 || m->up_fold[pc] >= 0)
            continue;
        const AexrtConv2DDesc d = desc_of(e.commands[pc]);
        if (d.kernel_h != 1 || d.kernel_w != 1 || is_f32(m, cs.out_value)) continue;
        m->up_fold[pc] = (int)ci;
        m->up_fold[ci] = pc;
    }
}

// Fills conv p's upsampled input source from resize ci: the resize's input,
// read at half resolution for the channels of its output's slice.
void set_upsampled_input(AexrtYoloModel* m, ConvParams& p, int ci) {
    const EngineCommand& rc = m->eng.commands[ci];
    const ValueInfo& o = m->vals[rc.output];
    const AexrtHipTensorView sv = view_of(m, (int)rc.inputs[0]);
    p.xup = sv.data;
    p.xup_nstride = sv.n_stride;
    p.xup_cstride = (int32_t)sv.c_stride;
    p.xup_c0 = (int32_t)o.pl.offset;
    p.xup_cn = o.C;
    p.xup_slots = slot_ref(sv);
    p.xup_nslots = o.C / 16;
}

// Writes the upsamples that folded convs read from their sources into their
// concat slices (synchronously), for reads of those values outside a run.
bool store_folded_upsamples(AexrtYoloModel* m, int root) {
    const Engine& e = m->eng;
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        if (e.commands[ci].kind != kCmdResize || m->up_read.size() <= ci || m->up_read[ci] < 0) continue;
        const ValueInfo& x = m->vals[e.commands[ci].inputs[0]];
        const ValueInfo& o = m->vals[e.commands[ci].output];
        if (o.pl.root != root) continue;
        const AexrtHipTensorView xv = view_of(m, (int)e.commands[ci].inputs[0]), yv = view_of(m, (int)e.commands[ci].output);
        if (!check_hip(launch_resize_nearest_nhwc(static_cast<const __half*>(xv.data), xv.n_stride, xv.c_stride,
                                                  static_cast<__half*>(yv.data), yv.n_stride, yv.c_stride, x.N, x.H,
                                                  x.W, x.C, o.H, o.W, SlotRef{nullptr, 1u, 0u}, m->stream),
                       "store upsample") ||
            !check_hip(hipStreamSynchronize(m->stream), "store upsample sync"))
            return false;
    }
    return true;
}

bool build_steps(AexrtYoloModel* m, const std::vector<CopyJob>& copies) {
    Engine& e = m->eng;
    auto& V = m->vals;
    m->steps.clear();
    m->chain_steps.clear();
    m->step_ms.clear();  // list scheduling measures the new steps again
    m->tunables.clear();
    setup_upsample_folds(m);
    {
        uint32_t* slots = m->slots;
        const int64_t n = int64_t(kSlotStripes) * m->slot_stride;
        m->steps.push_back(Step{-1, "amax slots clear " + std::to_string(n) + " words", [slots, n](hipStream_t s) {
                                    return launch_fill_u32(slots, n, 0u, s);
                                }});
        m->steps.back().all = true;
    }
    {
        int npairs = 0;
        for (const ConvState& cs : m->convs) npairs += cs.pair_b >= 0 && is_int8_algorithm(cs.algorithm) ? 1 : 0;
        if (npairs > m->n_pair_sync) {
            m->pair_sync = static_cast<uint32_t*>(dev_alloc(m, (size_t)npairs * kPairSyncWordsHost * 4));
            if (!m->pair_sync) return fail(m, "out of device memory for superblock sync words");
            m->n_pair_sync = npairs;
        }
        if (npairs > 0 && !m->pair_err) {
            m->pair_err = static_cast<uint32_t*>(dev_alloc(m, 256));
            if (!m->pair_err || hipMemset(m->pair_err, 0, 256) != hipSuccess)
                return fail(m, "out of device memory for the superblock error word");
        }
        if (npairs > 0) {
            uint32_t* sync = m->pair_sync;
            const int64_t n = (int64_t)npairs * kPairSyncWordsHost;
            m->steps.push_back(Step{-1, "superblock sync clear " + std::to_string(n) + " words", [sync, n](hipStream_t s) {
                                        return launch_fill_u32(sync, n, 0u, s);
                                    }});
            m->steps.back().all = true;
        }
    }
    int pair_k = 0;  // int8 superblock steps built so far (their sync areas)
    const uint32_t in_v = e.manifest.input_value;
    if (m->input_needs_nhwc) {
        const ValueInfo& x = V[in_v];
        AexrtHipTensorView y = view_of(m, (int)in_v);
        const float* src = m->input_dev;
        const int N = x.N, C = x.C, HW = x.H * x.W;
        if (x.cpad > x.C) {
            m->steps.push_back(Step{-1, "input nchw->nhwc8", [=](hipStream_t s) {
                                        return launch_nchw_f32_to_nhwc8(src, static_cast<__half*>(y.data), N, C, HW, s);
                                    }});
            m->steps.back().writes = {V[in_v].pl.root};
        } else {
            m->steps.push_back(Step{-1, "input nchw->nhwc", [=](hipStream_t s) {
                                        return launch_nchw_f32_to_nhwc_f16(src, static_cast<__half*>(y.data),
                                                                           y.n_stride, y.c_stride, N, C, HW,
                                                                           slot_ref(y), s);
                                    }});
            m->steps.back().writes = {V[in_v].pl.root};
        }
    }
    std::vector<bool> done(e.commands.size(), false);  // folded into an earlier step
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        if (done[ci]) continue;
        switch (c.kind) {
            case kCmdConv:
            case kCmdConvSilu: {
                ConvState& cs = m->convs[ci];
                const int xv = (int)c.inputs[0];
                AexrtConv2DDesc d = conv_desc_padded(m, ci);
                // a sibling pair whose weights still are those the pair was built from
                const int sib = m->sibling.empty() ? -1 : m->sibling[ci];
                if (cs.chain_b >= 0) {
                    bool built = false;
                    if (!build_chain_step(m, ci, done, built)) return false;
                    if (built) break;
                }
                if (cs.pair_b >= 0) {
                    bool built = false;
                    const bool int8_pair = is_int8_algorithm(cs.algorithm);
                    if (!build_pair_step(m, ci, pair_k, done, built)) return false;
                    if (built) {
                        if (int8_pair) ++pair_k;
                        break;
                    }
                }
                const bool pair = m->merge_siblings && sib >= 0 && !done[sib] && cs.w_pair && cs.pair_src[0] == cs.w &&
                                  cs.pair_src[1] == m->convs[sib].w && cs.chain_b < 0 && m->convs[sib].chain_b < 0;
                if (pair) d.out_channels += desc_of(e.commands[sib]).out_channels;
                uint32_t flags = c.kind == kCmdConvSilu ? AEXRT_HIP_CONV_SILU : 0u;
                AexrtHipTensorView xvw{};
                if (m->vals[xv].is_input && m->input_nchw_direct) {
                    const ValueInfo& xi = m->vals[xv];
                    xvw.data = m->input_dev;
                    xvw.n_stride = int64_t(xi.C) * xi.H * xi.W;
                    xvw.c_stride = xi.C;
                    flags |= AEXRT_HIP_CONV_IN_NCHW_F32;
                } else {
                    xvw = view_of(m, xv);
                }
                const int yv = cs.out_value;
                AexrtHipTensorView yvw = view_of(m, yv);
                if (is_f32(m, yv)) flags |= AEXRT_HIP_CONV_OUT_F32;
                AexrtHipTensorView rvw{};
                if (cs.fused_residual) {
                    flags |= AEXRT_HIP_CONV_RESIDUAL;
                    rvw = view_of(m, cs.residual_value);
                }
                // pg16: group g's scale comes from the reference's memory strip
                // g of the NCHW tensor, which is channel group g at N = 1 (the
                // input's own slots); at N > 1 the strips mix images and are
                // taken by a separate pass into a buffer of this conv
                AexrtHipTensorView strip_src{};
                int strip_n = 0, strip_hw = 0, strip_c = 0;
                if (cs.pg16) {
                    flags |= AEXRT_HIP_CONV_INT8_PG16;
                    if (d.batch > 1) {
                        strip_src = xvw;
                        strip_n = (int)d.batch;
                        strip_hw = (int)(d.in_h * d.in_w);
                        strip_c = (int)d.in_channels;
                        cs.strips = static_cast<uint32_t*>(dev_alloc(m, d.in_channels / 16 * 4));
                        if (!cs.strips) return fail(m, "out of device memory for pg16 strips");
                        xvw.amax_slots = cs.strips;
                        xvw.amax_stripes = 1;
                        xvw.amax_stripe_stride = 0;
                    }
                }
                // a9: the reference quantizes an int8 conv's input per (position,
                // 4 channels) in the kernel when the input has fewer than 4096
                // elements (RT:21478-21479); otherwise a per-tensor int8 conv whose
                // input slots do not cover every channel takes its own amax pass
                const bool int8 = is_int8_algorithm(cs.algorithm);
                AexrtHipTensorView own_src{};
                bool own_pass = false;
                if (int8 && cs.dynamic) {
                    flags |= AEXRT_HIP_CONV_INT8_DYNAMIC;
                } else if (int8 && !cs.pg16 && (!xvw.amax_slots || !m->roots[V[xv].pl.root].slots_complete)) {
                    if (!cs.own_slots) cs.own_slots = static_cast<uint32_t*>(dev_alloc(m, d.in_channels / 16 * 4));
                    if (!cs.own_slots) return fail(m, "out of device memory for conv amax slots");
                    own_src = xvw;
                    xvw.amax_slots = cs.own_slots;
                    xvw.amax_stripes = 1;
                    xvw.amax_stripe_stride = 0;
                    own_pass = true;
                }
                ConvParams p{};
                std::string why;
                if (!build_conv_params(d, cs.algorithm, flags, xvw, pair ? cs.w_pair : cs.w, cs.scale,
                                       pair ? cs.bias_pair : cs.bias, cs.fused_residual ? &rvw : nullptr, yvw, nullptr,
                                       p, why))
                    return fail(m, "command " + std::to_string(ci) + ": " + why);
                if (m->up_read[ci] >= 0) {
                    set_upsampled_input(m, p, m->up_read[ci]);
                    if (own_pass) return fail(m, "command " + std::to_string(ci) + ": upsampled input without slots");
                }
                int upv = -1;  // output value of a resize folded into this conv
                if (m->up_fold[ci] >= 0) {
                    const EngineCommand& rc = e.commands[m->up_fold[ci]];
                    const AexrtHipTensorView uv = view_of(m, (int)rc.output);
                    p.yup = uv.data;
                    p.yup_nstride = uv.n_stride;
                    p.yup_cstride = (int32_t)uv.c_stride;
                    p.yup_slots = slot_ref(uv);
                    ConvChoice probe[4];
                    if (own_pass || enumerate_conv_choices(p, int8, probe, 4) == 0) {
                        p.yup = nullptr;  // the kernel does not take it: the resize runs
                        m->up_fold[m->up_fold[ci]] = -1;
                        m->up_fold[ci] = -1;
                    } else {
                        upv = (int)rc.output;
                    }
                }
                int f2v = -1;  // output value of a 1x1 conv fused into this conv's epilogue
                if (cs.fused_1x1 >= 0) {
                    // fused only where a 32x32-MFMA tile holds every output channel of the
                    // 3x3 conv (its resident weights and windows fit LDS); otherwise both
                    // convs run on their own and the 3x3 output is stored
                    ConvParams probe = p;
                    ConvParams probe2 = p;
                    probe2.C = (int)d.out_channels;
                    probe2.OC = (int)desc_of(e.commands[cs.fused_1x1]).out_channels;
                    probe2.OCp = (probe2.OC + 15) / 16 * 16;
                    probe2.Kp = (probe2.C + 63) / 64 * 64;
                    probe2.KH = probe2.KW = 1;
                    probe2.S = 1;
                    probe2.P = 0;
                    probe2.H = p.OH;
                    probe2.W = p.OW;
                    probe2.flags = 0;
                    probe.fuse_1x1 = &probe2;
                    ConvChoice none[4];
                    if (enumerate_m32_choices(probe, false, none, 4) == 0) {
                        m->convs[cs.fused_1x1].fused_into = -1;
                        cs.fused_1x1 = -1;
                        V[c.output].elided = false;
                    }
                }
                if (cs.fused_1x1 >= 0) {
                    const int cj = cs.fused_1x1;
                    const ConvState& cn = m->convs[cj];
                    const EngineCommand& n = e.commands[cj];
                    const uint32_t flags2 = (n.kind == kCmdConvSilu ? AEXRT_HIP_CONV_SILU : 0u) |
                                            (is_f32(m, cn.out_value) ? AEXRT_HIP_CONV_OUT_F32 : 0u);
                    if (!build_conv_params(conv_desc_padded(m, cj), cn.algorithm, flags2, yvw, cn.w, nullptr, cn.bias,
                                           nullptr, view_of(m, cn.out_value), nullptr, cs.f2p, why))
                        return fail(m, "command " + std::to_string(cj) + " (fused 1x1): " + why);
                    p.fuse_1x1 = &cs.f2p;
                    f2v = cn.out_value;
                    done[cj] = true;
                }
                const uint32_t alg = cs.algorithm;
                std::function<hipError_t(hipStream_t)> pre;
                if (own_pass) {
                    uint32_t* own = cs.own_slots;
                    const int on = (int)d.batch, ohw = (int)(d.in_h * d.in_w), oc_in = (int)d.in_channels;
                    pre = [=](hipStream_t s) {
                        hipError_t e = launch_fill_u32(own, oc_in / 16, 0u, s);
                        if (e == hipSuccess)
                            e = launch_amax_slots_nhwc(static_cast<const __half*>(own_src.data), own_src.n_stride,
                                                       own_src.c_stride, on, ohw, oc_in, SlotRef{own, 1u, 0u}, s);
                        return e;
                    };
                }
                std::string head = conv_label(c, e.src_cmd[ci], alg);
                std::function<std::string()> family;
                if (cs.pg16) {
                    uint32_t* strips = cs.strips;
                    m->steps.push_back(Step{(int)ci, "", [=](hipStream_t s) {
                                                if (strips) {
                                                    hipError_t e = launch_fill_u32(strips, strip_c / 16, 0u, s);
                                                    if (e == hipSuccess)
                                                        e = launch_amax_strips_nhwc(
                                                            static_cast<const __half*>(strip_src.data),
                                                            strip_src.n_stride, strip_src.c_stride, strip_n,
                                                            strip_hw, strip_c, strips, s);
                                                    if (e != hipSuccess) return e;
                                                }
                                                return launch_conv_int8_pg16(p, s);
                                            }});
                    head += " pg16";
                    family = [] { return std::string("conv_int8_pg16_kernel"); };
                } else if (int8 && cs.dynamic) {
                    const DynConvParams dp = dynamic_params(p);
                    m->steps.push_back(Step{(int)ci, "", [dp](hipStream_t s) { return launch_conv_int8_dynamic(dp, s); }});
                    head += " dynamic";
                    family = [] { return std::string("conv_int8_dynamic_kernel"); };
                } else if (m->autotune && !is_winograd_algorithm(alg)) {
                    auto tc = std::make_unique<TunedConv>();
                    tc->cmd = (int)ci;
                    tc->int8 = int8;
                    if (!tune_conv(m, p, tc->int8, &tc->cands)) return false;
                    tc->key = refined_key(ci, alg, p, tc->int8);
                    auto rf = m->refined.find(tc->key);
                    if (rf != m->refined.end()) {
                        for (const ConvChoice& k : tc->cands) tc->done = tc->done || same_choice(k, rf->second);
                        if (!tc->done) {
                            // a choice of an earlier measurement in the network: kept when this
                            // build still offers it for the conv
                            std::vector<ConvChoice> all(kMaxConvChoices);
                            const int na = enumerate_conv_choices(p, tc->int8, all.data(), kMaxConvChoices);
                            for (int k = 0; k < na; ++k) tc->done = tc->done || same_choice(all[k], rf->second);
                        }
                        if (tc->done) p.choice = rf->second;
                    }
                    tc->p = p;
                    tc->step = m->steps.size();
                    TunedConv* t = tc.get();
                    m->tunables.push_back(std::move(tc));
                    m->steps.push_back(Step{(int)ci, "", [t, pre](hipStream_t s) {
                                                if (pre) {
                                                    const hipError_t e = pre(s);
                                                    if (e != hipSuccess) return e;
                                                }
                                                return launch_conv_igemm(t->p, t->int8, s);
                                            }});
                    family = [t] {
                        char name[96];
                        conv_kernel_name(t->p, t->int8, name, sizeof(name));
                        return std::string(name);
                    };
                    if (int8) m->steps.back().conv_params = [t] { return t->p; };
                } else {
                    if (!is_winograd_algorithm(alg)) apply_cached_choice(m, ci, alg, p, int8);
                    m->steps.push_back(Step{(int)ci, "", [p, alg, pre](hipStream_t s) {
                                                if (pre) {
                                                    const hipError_t e = pre(s);
                                                    if (e != hipSuccess) return e;
                                                }
                                                if (is_winograd_algorithm(alg)) return launch_winograd_f2x2(p, s);
                                                return launch_conv_igemm(p, is_int8_algorithm(alg), s);
                                            }});
                    if (is_winograd_algorithm(alg)) {
                        family = [] { return std::string("winograd_f2x2_kernel"); };
                    } else {
                        family = [p, int8] {
                            char name[96];
                            conv_kernel_name(p, int8, name, sizeof(name));
                            return std::string(name);
                        };
                        if (int8) m->steps.back().conv_params = [p] { return p; };
                    }
                }
                if (own_pass) head += " own-amax";
                Step& st = m->steps.back();
                st.head = head;
                st.family = family;
                if (!(m->vals[xv].is_input && m->input_nchw_direct)) st.reads.push_back(V[xv].pl.root);
                if (cs.fused_residual) st.reads.push_back(V[cs.residual_value].pl.root);
                st.writes = {V[f2v >= 0 ? f2v : yv].pl.root};
                if (f2v >= 0) st.tail = " then 1x1 cmd#" + std::to_string(e.src_cmd[cs.fused_1x1]);
                if (upv >= 0) {
                    st.writes.push_back(V[upv].pl.root);
                    st.tail = " + 2x upsample cmd#" + std::to_string(e.src_cmd[m->up_fold[ci]]);
                }
                if (m->up_read[ci] >= 0) {
                    st.reads.push_back(V[e.commands[m->up_read[ci]].inputs[0]].pl.root);
                    st.tail = " reading 2x upsample cmd#" + std::to_string(e.src_cmd[m->up_read[ci]]);
                }
                if (pair) {
                    done[sib] = true;
                    st.tail = " + cmd#" + std::to_string(e.src_cmd[sib]);
                }
                break;
            }
            case kCmdConcat: {
                for (const CopyJob& j : copies) {
                    if (j.cmd != (int)ci) continue;
                    const ValueInfo& x = V[j.src];
                    if (is_f32(m, j.src) || m->roots[j.dst.root].f32)
                        return fail(m, "command " + std::to_string(ci) + ": fp32 concat copy is not supported");
                    AexrtHipTensorView s = view_of(m, j.src), dv = view_of_pl(m, j.dst);
                    if (x.C % 8) return fail(m, "command " + std::to_string(ci) + ": concat copy needs C % 8 == 0");
                    const int N = x.N, HW = x.H * x.W, C = x.C;
                    m->steps.push_back(Step{(int)ci, "cmd#" + std::to_string(e.src_cmd[ci]) + " CONCAT copy", [=](hipStream_t st) {
                                                return launch_copy_nhwc(static_cast<const __half*>(s.data), s.n_stride,
                                                                        s.c_stride, static_cast<__half*>(dv.data),
                                                                        dv.n_stride, dv.c_stride, N, HW, C,
                                                                        slot_ref(dv), st);
                                            }});
                    m->steps.back().reads = {V[j.src].pl.root};
                    m->steps.back().writes = {j.dst.root};
                }
                break;
            }
            case kCmdMaxpool: {
                const ValueInfo& x = V[c.inputs[0]];
                const ValueInfo& o = V[c.output];
                // SPPF: three chained 5x5 / s1 / p2 pools run as one kernel
                auto sppf_link = [&](size_t k, uint32_t in) {
                    if (k >= e.commands.size()) return false;
                    const EngineCommand& d = e.commands[k];
                    return d.kind == kCmdMaxpool && d.inputs[0] == in && d.params[6] == 5 && d.params[8] == 1 &&
                           d.params[10] == 2 && V[d.output].H == x.H && V[d.output].W == x.W;
                };
                if (sppf_link(ci, c.inputs[0]) && sppf_link(ci + 1, c.output) &&
                    sppf_link(ci + 2, e.commands[ci + 1].output) && x.C % 16 == 0 && sppf_fits(x.H, x.W)) {
                    const int v1 = (int)c.output, v2 = (int)e.commands[ci + 1].output,
                              v3 = (int)e.commands[ci + 2].output;
                    AexrtHipTensorView xv = view_of(m, (int)c.inputs[0]), a = view_of(m, v1), b = view_of(m, v2),
                                       d = view_of(m, v3);
                    if (a.n_stride == b.n_stride && a.n_stride == d.n_stride && a.c_stride == b.c_stride &&
                        a.c_stride == d.c_stride) {
                        const int N = x.N, H = x.H, W = x.W, C = x.C;
                        m->steps.push_back(Step{(int)ci, "cmd#" + std::to_string(e.src_cmd[ci]) + " SPPF MAXPOOL x3",
                                                [=](hipStream_t st) {
                                                    return launch_sppf_maxpool_nhwc(
                                                        static_cast<const __half*>(xv.data), xv.n_stride, xv.c_stride,
                                                        static_cast<__half*>(a.data), static_cast<__half*>(b.data),
                                                        static_cast<__half*>(d.data), a.n_stride, a.c_stride, N, H,
                                                        W, C, slot_ref(a), slot_ref(b), slot_ref(d), st);
                                                }});
                        m->steps.back().reads = {V[c.inputs[0]].pl.root};
                        m->steps.back().writes = {V[v1].pl.root, V[v2].pl.root, V[v3].pl.root};
                        done[ci + 1] = done[ci + 2] = true;
                        break;
                    }
                }
                AexrtHipTensorView xv = view_of(m, (int)c.inputs[0]), yv = view_of(m, (int)c.output);
                const int N = x.N, H = x.H, W = x.W, C = x.C, OH = o.H, OW = o.W;
                const int k = (int)c.params[6], st = (int)c.params[8], pad = (int)c.params[10];
                if (C % 8) return fail(m, "command " + std::to_string(ci) + ": MAXPOOL needs C % 8 == 0");
                m->steps.push_back(Step{(int)ci, "cmd#" + std::to_string(e.src_cmd[ci]) + " MAXPOOL", [=](hipStream_t s) {
                                            return launch_maxpool_nhwc(static_cast<const __half*>(xv.data), xv.n_stride,
                                                                       xv.c_stride, static_cast<__half*>(yv.data),
                                                                       yv.n_stride, yv.c_stride, N, H, W, C, OH, OW, k,
                                                                       st, pad, slot_ref(yv), s);
                                        }});
                m->steps.back().reads = {V[c.inputs[0]].pl.root};
                m->steps.back().writes = {V[c.output].pl.root};
                break;
            }
            case kCmdResize: {
                if (m->up_fold[ci] >= 0 || m->up_read[ci] >= 0) break;  // folded into a conv
                const ValueInfo& x = V[c.inputs[0]];
                const ValueInfo& o = V[c.output];
                AexrtHipTensorView xv = view_of(m, (int)c.inputs[0]), yv = view_of(m, (int)c.output);
                const int N = x.N, H = x.H, W = x.W, C = x.C, OH = o.H, OW = o.W;
                if (C % 8) return fail(m, "command " + std::to_string(ci) + ": RESIZE needs C % 8 == 0");
                m->steps.push_back(Step{(int)ci, "cmd#" + std::to_string(e.src_cmd[ci]) + " RESIZE", [=](hipStream_t s) {
                                            return launch_resize_nearest_nhwc(
                                                static_cast<const __half*>(xv.data), xv.n_stride, xv.c_stride,
                                                static_cast<__half*>(yv.data), yv.n_stride, yv.c_stride, N, H, W, C, OH,
                                                OW, slot_ref(yv), s);
                                        }});
                m->steps.back().reads = {V[c.inputs[0]].pl.root};
                m->steps.back().writes = {V[c.output].pl.root};
                break;
            }
            case kCmdBinary: {
                if (is_fused_add(m, ci)) break;
                const ValueInfo& o = V[c.output];
                AexrtHipTensorView av = view_of(m, (int)c.inputs[0]), bv = view_of(m, (int)c.inputs[1]),
                                   yv = view_of(m, (int)c.output);
                const int N = o.N, HW = o.H * o.W, C = o.C;
                if (C % 8) return fail(m, "command " + std::to_string(ci) + ": BINARY needs C % 8 == 0");
                m->steps.push_back(Step{(int)ci, "cmd#" + std::to_string(e.src_cmd[ci]) + " BINARY add", [=](hipStream_t s) {
                                            return launch_add_nhwc(static_cast<const __half*>(av.data), av.n_stride,
                                                                   av.c_stride, static_cast<const __half*>(bv.data),
                                                                   bv.n_stride, bv.c_stride,
                                                                   static_cast<__half*>(yv.data), yv.n_stride,
                                                                   yv.c_stride, N, HW, C, slot_ref(yv), s);
                                        }});
                m->steps.back().reads = {V[c.inputs[0]].pl.root, V[c.inputs[1]].pl.root};
                m->steps.back().writes = {V[c.output].pl.root};
                break;
            }
            default:
                break;  // VIEW / ALIAS: placement only
        }
    }
    label_steps(m);
    schedule_steps(m);
    return true;
}

void drop_graph(AexrtYoloModel* m) {
    if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->graph_exec = nullptr;
    m->graph = nullptr;
    m->graph_valid = false;
}

bool launch_steps(AexrtYoloModel* m, hipStream_t s) {
    for (const Step& st : m->steps) {
        hipError_t e = st.launch(s);
        if (e != hipSuccess) return fail(m, st.label + ": " + hipGetErrorString(e));
    }
    return true;
}

// Issues the steps over the lanes (lane 0 = s) inside a stream capture: the
// other lanes fork from s before the first step, wait on the events of their
// cross-lane dependencies, and s joins them all at the end.
bool launch_steps_lanes(AexrtYoloModel* m, hipStream_t s) {
    auto& st = m->steps;
    if (m->step_events.size() < st.size()) {
        size_t k = m->step_events.size();
        m->step_events.resize(st.size(), nullptr);
        for (; k < st.size(); ++k)
            if (!check_hip(hipEventCreateWithFlags(&m->step_events[k], hipEventDisableTiming), "step event"))
                return fail(m, last_error());
    }
    auto new_event = [&](hipEvent_t& e) {
        e = nullptr;
        if (!check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "lane event")) return false;
        m->lane_events.push_back(e);
        return true;
    };
    hipStream_t lanes[kLanes];
    lanes[0] = s;
    bool used[kLanes] = {};
    for (int l = 1; l < kLanes; ++l) lanes[l] = m->lane_stream[l];
    for (const Step& x : st) used[x.lane] = true;
    bool any = false;
    for (int l = 1; l < kLanes; ++l) any = any || used[l];
    hipEvent_t fork = nullptr;
    if (any && (!new_event(fork) || !check_hip(hipEventRecord(fork, s), "fork record"))) return fail(m, last_error());
    for (int l = 1; l < kLanes; ++l)
        if (used[l] && !check_hip(hipStreamWaitEvent(lanes[l], fork, 0), "fork wait")) return fail(m, last_error());
    for (size_t i = 0; i < st.size(); ++i) {
        const int l = st[i].lane;
        for (int d : st[i].deps)
            if (st[d].lane != l && !check_hip(hipStreamWaitEvent(lanes[l], m->step_events[d], 0), "step wait"))
                return fail(m, last_error());
        const hipError_t e = st[i].launch(lanes[l]);
        if (e != hipSuccess) return fail(m, st[i].label + ": " + hipGetErrorString(e));
        if (st[i].signal && !check_hip(hipEventRecord(m->step_events[i], lanes[l]), "step record"))
            return fail(m, last_error());
    }
    for (int l = 1; l < kLanes; ++l) {
        if (!used[l]) continue;
        hipEvent_t join = nullptr;
        if (!new_event(join) || !check_hip(hipEventRecord(join, lanes[l]), "join record") ||
            !check_hip(hipStreamWaitEvent(s, join, 0), "join wait"))
            return fail(m, last_error());
    }
    return true;
}

bool run_network(AexrtYoloModel* m, hipStream_t s) {
    if (m->profile) {
        // The steps are launched one by one with an event after each, twice
        // in a row; the second pass is the one timed: by then the stream holds
        // the first pass's work, so no step waits for the host to launch it.
        std::vector<hipEvent_t> ev(m->steps.size() + 1, nullptr);
        bool ok = true;
        for (auto& e : ev) ok = ok && check_hip(hipEventCreate(&e), "profile event create");
        if (!ok) fail(m, last_error());
        for (int pass = 0; pass < 2 && ok; ++pass) {
            if (pass == 1) ok = check_hip(hipEventRecord(ev[0], s), "profile event record");
            for (size_t i = 0; i < m->steps.size() && ok; ++i) {
                hipError_t e = m->steps[i].launch(s);
                if (e != hipSuccess) ok = fail(m, m->steps[i].label + ": " + hipGetErrorString(e));
                else if (pass == 1 && !check_hip(hipEventRecord(ev[i + 1], s), "profile event record"))
                    ok = fail(m, last_error());
            }
        }
        if (ok && !check_hip(hipEventSynchronize(ev.back()), "profile sync")) ok = fail(m, last_error());
        m->prof_labels.clear();
        m->prof_ms.clear();
        for (size_t i = 0; ok && i < m->steps.size(); ++i) {
            float ms = 0.f;
            if (!check_hip(hipEventElapsedTime(&ms, ev[i], ev[i + 1]), "profile elapsed")) {
                ok = fail(m, last_error());
                break;
            }
            m->prof_labels.push_back(m->steps[i].label);
            m->prof_ms.push_back(ms);
        }
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        return ok;
    }
    if (!m->use_graph) return launch_steps(m, s);
    if (!m->graph_valid) {
        drop_graph(m);
        if (!check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "graph capture begin"))
            return fail(m, last_error());
        const bool ok = launch_steps_lanes(m, s);
        hipGraph_t g = nullptr;
        const hipError_t ec = hipStreamEndCapture(s, &g);
        if (!ok) {
            if (g) (void)hipGraphDestroy(g);
            return false;
        }
        if (ec != hipSuccess) return fail(m, std::string("graph capture end: ") + hipGetErrorString(ec));
        m->graph = g;
        if (!check_hip(hipGraphInstantiate(&m->graph_exec, g, nullptr, nullptr, 0), "graph instantiate"))
            return fail(m, last_error());
        m->graph_valid = true;
    }
    return check_hip(hipGraphLaunch(m->graph_exec, s), "graph launch") ? true : fail(m, last_error());
}

// The isolated measurement of tune_conv runs a conv back to back on its own
// buffers, with its input, output and weights warm in L2 and the MALL; in the
// network the input was just written by another kernel and the weights are
// cold, and the fastest isolated choice is often not the fastest there.
// Every conv's kContextCands fastest isolated candidates are therefore timed
// again inside the network: in round r each conv runs its r-th candidate, the
// steps are launched one by one between events (one warm-up pass, then
// kContextReps passes, the minimum per step counts), and each conv keeps the
// candidate with its shortest step.
constexpr int kContextReps = 3;

bool profiled_step_times(AexrtYoloModel* m, std::vector<float>& lo);
bool choose_chain_tiles(AexrtYoloModel* m);

bool refine_candidates(AexrtYoloModel* m) {
    size_t rounds = 0;
    for (const auto& t : m->tunables)
        if (!t->done && t->cands.size() > 1) rounds = std::max(rounds, t->cands.size());
    if (rounds == 0) return true;
    std::vector<std::vector<float>> ms(m->tunables.size());
    const bool prof = m->profile;
    m->profile = true;
    bool ok = true;
    for (size_t r = 0; r < rounds && ok; ++r) {
        for (auto& t : m->tunables)
            if (!t->done && !t->cands.empty()) t->p.choice = t->cands[std::min(r, t->cands.size() - 1)];
        std::vector<float> lo(m->steps.size(), 1e30f);
        for (int rep = 0; rep <= kContextReps && ok; ++rep) {
            ok = run_network(m, m->stream);
            for (size_t i = 0; ok && rep > 0 && i < m->steps.size() && i < m->prof_ms.size(); ++i)
                lo[i] = std::min(lo[i], (float)m->prof_ms[i]);
        }
        for (size_t k = 0; ok && k < m->tunables.size(); ++k) ms[k].push_back(lo[m->tunables[k]->step]);
    }
    m->profile = prof;
    m->prof_labels.clear();
    m->prof_ms.clear();
    if (!ok) return false;
    for (size_t k = 0; k < m->tunables.size(); ++k) {
        TunedConv& t = *m->tunables[k];
        if (t.done || t.cands.empty()) continue;
        size_t bi = 0;
        for (size_t r = 1; r < t.cands.size(); ++r)
            if (ms[k][r] < ms[k][bi]) bi = r;
        t.p.choice = t.cands[bi];
        t.done = true;
        m->refined[t.key] = t.p.choice;
        if (m->tune_log)
            std::fprintf(stderr, "aexrt in-network %s: candidate %zu of %zu  %.2f us (first %.2f us)\n",
                         m->steps[t.step].label.c_str(), bi, t.cands.size(), ms[k][bi] * 1000.0f, ms[k][0] * 1000.0f);
    }
    label_steps(m);
    drop_graph(m);
    return true;
}

bool refine_in_context(AexrtYoloModel* m) { return refine_candidates(m) && choose_chain_tiles(m); }

// The tile of each chain launch not measured yet: the tiles the kernel offers
// for it (whole map, halves, thirds, 8x8 down to 3x3) timed in the network
// like the conv candidates above (round r: every chain on its r-th tile, the
// least of kContextReps event-profiled passes per step), the fastest kept.  A
// small batch has few tiles of the whole map (one block per image and
// branch), and smaller tiles spread the chain over more of the GPU at the cost
// of recomputing their borders; a large batch keeps the large tiles.
bool choose_chain_tiles(AexrtYoloModel* m) {
    struct Todo {
        size_t k;
        std::vector<std::pair<int, int>> tiles;
    };
    std::vector<Todo> todo;
    size_t rounds = 0;
    for (size_t k = 0; k < m->chain_steps.size(); ++k) {
        auto& c = m->chain_steps[k];
        if (c.done) continue;
        ConvParams br0[3], br1[3];
        int tr[16], tc[16];
        int n = 0;
        if (chain_params_of(m, c.ci, br0) && (c.partner < 0 || chain_params_of(m, (size_t)c.partner, br1)))
            n = enumerate_chain_tiles(br0, c.partner >= 0 ? br1 : nullptr, tr, tc, 16);
        if (n <= 1) {
            c.done = true;
            continue;
        }
        Todo t{k, {}};
        for (int i = 0; i < n; ++i) t.tiles.emplace_back(tr[i], tc[i]);
        rounds = std::max(rounds, t.tiles.size());
        todo.push_back(std::move(t));
    }
    if (todo.empty()) return true;
    std::vector<std::vector<float>> ms(todo.size());
    for (size_t r = 0; r < rounds; ++r) {
        for (const Todo& t : todo) {
            const auto& tile = t.tiles[std::min(r, t.tiles.size() - 1)];
            ConvState& cs = m->convs[m->chain_steps[t.k].ci];
            cs.chain_tr = tile.first;
            cs.chain_tc = tile.second;
        }
        std::vector<float> lo;
        if (!profiled_step_times(m, lo)) return false;
        for (size_t i = 0; i < todo.size(); ++i) {
            const size_t st = m->chain_steps[todo[i].k].step;
            ms[i].push_back(st < lo.size() ? lo[st] : 1e30f);
        }
    }
    for (size_t i = 0; i < todo.size(); ++i) {
        auto& c = m->chain_steps[todo[i].k];
        size_t bi = 0;
        for (size_t r = 1; r < todo[i].tiles.size(); ++r)
            if (ms[i][r] < ms[i][bi]) bi = r;
        ConvState& cs = m->convs[c.ci];
        cs.chain_tr = todo[i].tiles[bi].first;
        cs.chain_tc = todo[i].tiles[bi].second;
        c.done = true;
        ConvChoice rec{};
        rec.tr = cs.chain_tr;
        rec.tc = cs.chain_tc;
        m->refined[c.key] = rec;
        if (m->tune_log)
            std::fprintf(stderr, "aexrt chain tile of %s: %dx%d, %zu of %zu  %.2f us (largest %.2f us)\n",
                         m->steps[c.step].label.c_str(), cs.chain_tr, cs.chain_tc, bi, todo[i].tiles.size(),
                         ms[i][bi] * 1000.0f, ms[i][0] * 1000.0f);
    }
    label_steps(m);
    drop_graph(m);
    return true;
}

// Per head 3x3 + 1x1 pair of m->fuse_pairs, the time of the steps of the current
// build that compute it: the fused step, or the 3x3 step plus the 1x1 step
// (the least of kContextReps event-profiled passes per step).
// Each step's time in the network, launched one by one between events: the
// least of kContextReps passes after a warm-up pass.
bool profiled_step_times(AexrtYoloModel* m, std::vector<float>& lo) {
    lo.assign(m->steps.size(), 1e30f);
    const bool prof = m->profile;
    m->profile = true;
    bool ok = true;
    for (int rep = 0; rep <= kContextReps && ok; ++rep) {
        ok = run_network(m, m->stream);
        for (size_t i = 0; ok && rep > 0 && i < m->steps.size() && i < m->prof_ms.size(); ++i)
            lo[i] = std::min(lo[i], (float)m->prof_ms[i]);
    }
    m->profile = prof;
    m->prof_labels.clear();
    m->prof_ms.clear();
    return ok;
}

bool pair_step_times(AexrtYoloModel* m, std::vector<float>& out) {
    out.assign(m->fuse_pairs.size(), 0.0f);
    if (m->fuse_pairs.empty()) return true;
    std::vector<float> lo;
    if (!profiled_step_times(m, lo)) return false;
    for (size_t k = 0; k < m->fuse_pairs.size(); ++k)
        for (size_t i = 0; i < m->steps.size(); ++i)
            if (m->steps[i].cmd == m->fuse_pairs[k].first || m->steps[i].cmd == m->fuse_pairs[k].second)
                out[k] += lo[i];
    return true;
}

// Spreading independent steps over streams pays when kernels are long enough to
// overlap (large batch) and costs cross-queue synchronization when they are not
// (batch 1): both schedules are captured and timed at load, the faster one kept.
// Time of 10 runs of the current schedule: the least of three such
// measurements after the graph is captured and warmed up.
bool time_schedule(AexrtYoloModel* m, float* ms_out) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!check_hip(hipEventCreate(&e0), "timing event") || !check_hip(hipEventCreate(&e1), "timing event")) {
        if (e0) (void)hipEventDestroy(e0);
        return fail(m, last_error());
    }
    drop_graph(m);
    bool ok = true;
    for (int r = 0; r < 5 && ok; ++r) ok = run_network(m, m->stream);  // capture + warm-up
    float best = 0.0f;
    for (int rep = 0; rep < 3 && ok; ++rep) {
        ok = check_hip(hipEventRecord(e0, m->stream), "timing record");
        for (int r = 0; r < 10 && ok; ++r) ok = run_network(m, m->stream);
        ok = ok && check_hip(hipEventRecord(e1, m->stream), "timing record") &&
             check_hip(hipEventSynchronize(e1), "timing sync");
        float ms = 0.0f;
        ok = ok && check_hip(hipEventElapsedTime(&ms, e0, e1), "timing elapsed");
        if (ok && (rep == 0 || ms < best)) best = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms_out = best;
    return ok;
}

// Schedules the current steps anew under the current lane count and policy; list
// scheduling measures the steps' times first when the step list changed since.
bool reschedule(AexrtYoloModel* m) {
    if (m->lane_policy == 1 && m->n_lanes > 1 && m->step_ms.size() != m->steps.size() &&
        !profiled_step_times(m, m->step_ms))
        return false;
    schedule_steps(m);
    drop_graph(m);
    return true;
}

// The fastest lane count of kLanes down to one, each under the dependency rule
// and under list scheduling (its time of 10 runs in *best_ms).
bool choose_lanes(AexrtYoloModel* m, float* best_ms) {
    *best_ms = 0.0f;
    if (!m->use_graph) return true;
    if (!profiled_step_times(m, m->step_ms)) return false;
    int best = 1, best_policy = 0;
    bool first = true;
    for (int policy = 0; policy < 2; ++policy)
        for (int lanes = kLanes; lanes >= (policy ? 2 : 1); --lanes) {
            if (m->lane_policy_forced >= 0 && policy != m->lane_policy_forced && lanes > 1) continue;
            m->n_lanes = lanes;
            m->lane_policy = policy;
            schedule_steps(m);
            float ms = 0.0f;
            if (!time_schedule(m, &ms)) return false;
            if (first || ms < *best_ms) {
                *best_ms = ms;
                best = lanes;
                best_policy = policy;
            }
            first = false;
        }
    m->n_lanes = best;
    m->lane_policy = best_policy;
    schedule_steps(m);
    drop_graph(m);
    if (m->tune_log)
        std::fprintf(stderr, "aexrt lanes: %d, %s (%.1f us per run)\n", best,
                     best_policy ? "list scheduled" : "dependency rule", *best_ms * 100.0f);
    return true;
}

// The manifest's YOLO head description (channels, anchors, classes,
// objectness) must match the network output for the postprocess to run:
// either a decoded output0 (4 box values, optional objectness, class
// scores) or the raw Detect head (64 DFL bin logits + class logits over the
// stride-8/16/32 grids of the input); any other output keeps output0 only.
void setup_postprocess(AexrtYoloModel* m) {
    const EngineManifest& mf = m->eng.manifest;
    const ValueInfo& o = m->vals[mf.output_value];
    const uint32_t cls_off = mf.has_objectness ? 5u : 4u;
    m->post_ok = o.known && o.pl.valid && o.rank == 3 && m->roots[o.pl.root].f32 && mf.classes > 0 &&
                 mf.channels == (uint32_t)o.C && mf.anchors == (uint32_t)o.H && mf.max_candidates >= 1 &&
                 mf.max_candidates <= (uint32_t)kYoloMaxCandidates && mf.max_detections >= 1;
    if (!m->post_ok) return;
    m->post_dfl = false;
    if (mf.channels != mf.classes + cls_off) {
        const ValueInfo& in = m->vals[mf.input_value];
        YoloLevels lv{};
        lv.n = 3;
        int total = 0;
        for (int l = 0; l < 3; ++l) {
            const int st = 8 << l;
            lv.h[l] = in.H / st;
            lv.w[l] = in.W / st;
            lv.stride[l] = (float)st;
            total += lv.h[l] * lv.w[l];
        }
        m->post_ok = !mf.has_objectness && mf.channels == mf.classes + 64 && in.H % 32 == 0 && in.W % 32 == 0 &&
                     total == (int)mf.anchors;
        if (!m->post_ok) return;
        m->post_dfl = true;
        m->post_levels = lv;
    }
    m->dets_dev = static_cast<float*>(dev_alloc(m, size_t(mf.max_detections) * 6 * 4));
    m->det_count_dev = static_cast<uint32_t*>(dev_alloc(m, 256));
    m->post_ok = m->dets_dev && m->det_count_dev;
}

bool launch_postprocess(AexrtYoloModel* m, hipStream_t s) {
    const EngineManifest& mf = m->eng.manifest;
    const AexrtHipTensorView ov = view_of(m, (int)mf.output_value);
    // image 0 of output0, element (channel, anchor) at anchor * c_stride + channel
    return check_hip(launch_yolo_decode_nms_topk(static_cast<const float*>(ov.data), 1, ov.c_stride, (int)mf.anchors,
                                                 (int)mf.classes, (int)mf.has_objectness, mf.conf_threshold,
                                                 mf.iou_threshold, (int)mf.max_candidates, (int)mf.max_detections,
                                                 m->dets_dev, m->det_count_dev, s,
                                                 m->post_dfl ? &m->post_levels : nullptr),
                     "yolo postprocess");
}

// The reference's prepared-plan counters (RT:29204-29285, 22913-23110) for this
// step list: engine commands without a launch of their own, the fusions
// performed, and the convs by the kernel family that runs them (the
// reference's "tileflow" buckets: 1x1 convs; 3x3 convs on a spatial tile
// kernel (halo window, wide, band); 3x3 dot4 convs (pack4: the dynamic int8
// kernel); 3x3 implicit-GEMM convs (igemm, pg16, Winograd) with their
// 40x40/20x20/10x10 and exact-shape sub-counts; fp16 MFMA convs).
void compute_stats(AexrtYoloModel* m) {
    PlanStats st{};
    const Engine& e = m->eng;
    std::vector<uint8_t> launched(e.manifest.command_count, 0);
    std::vector<uint8_t> conv_kind(e.commands.size(), 0);  // 1 igemm, 2 spatial, 3 dot4
    for (const Step& x : m->steps) {
        if (x.cmd < 0) continue;
        if (e.src_cmd[x.cmd] < launched.size()) launched[e.src_cmd[x.cmd]] = 1;
        if (!x.family) continue;
        const std::string f = x.family();
        const uint8_t k = f.rfind("conv_int8_dynamic", 0) == 0 ? 3
                          : (f.rfind("conv3x3_halo", 0) == 0 || f.rfind("conv3x3_wide", 0) == 0 ||
                             f.rfind("conv3x3_stem", 0) == 0 || f.rfind("conv3x3_m32", 0) == 0 ||
                             f.rfind("conv_pair", 0) == 0)
                              ? 2
                              : 1;
        conv_kind[x.cmd] = k;
        if (x.tail.find("superblock") != std::string::npos) {
            ++st.c2f_superblocks;
            if (m->convs[x.cmd].pair_b >= 0) conv_kind[m->convs[x.cmd].pair_b] = k;
        }
        if (x.tail.rfind(" + cmd#", 0) == 0) {  // a sibling pair in one launch
            st.paired_conv3x3 += desc_of(e.commands[x.cmd]).kernel_h == 3;
            if (m->sibling[x.cmd] >= 0) conv_kind[m->sibling[x.cmd]] = k;
        }
    }
    for (uint8_t v : launched) st.skipped += v ? 0u : 1u;
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        const EngineCommand& c = e.commands[ci];
        if (c.kind == kCmdConcat) {
            bool copied = false;
            for (const CopyJob& j : m->copies) copied = copied || j.cmd == (int)ci;
            bool feeds_1x1 = false;
            for (int u : m->vals[c.output].consumers)
                feeds_1x1 = feeds_1x1 || (m->convs[u].is_conv && desc_of(e.commands[u]).kernel_h == 1);
            st.late_concat_conv1x1 += !copied && feeds_1x1;
        }
        const ConvState& cs = m->convs[ci];
        if (!cs.is_conv) continue;
        st.tail_residual += cs.fused_residual;
        st.head_final_conv += cs.fused_1x1 >= 0;
        st.native_fp16 += !is_int8_algorithm(cs.algorithm);
        const AexrtConv2DDesc d = desc_of(c);
        if (d.kernel_h == 1) {
            ++st.conv1x1;
            continue;
        }
        if (conv_kind[ci] == 2) {
            ++st.spatial3x3;
            continue;
        }
        if (conv_kind[ci] == 3) {
            ++st.pack4_3x3;
            continue;
        }
        ++st.igemm3x3;
        st.igemm3x3_40 += d.out_h == 40;
        st.igemm3x3_20 += d.out_h == 20;
        st.igemm3x3_10 += d.out_h == 10;
        const uint32_t ic = d.in_channels, oc = d.out_channels;
        st.exact_40_64x64 += d.out_h == 40 && ic == 64 && oc == 64;
        st.exact_20_64x64 += d.out_h == 20 && ic == 64 && oc == 64;
        st.exact_10_128x128 += d.out_h == 10 && ic == 128 && oc == 128;
        st.exact_20_128x64 += d.out_h == 20 && ic == 128 && oc == 64;
        st.exact_10_256x64 += d.out_h == 10 && ic == 256 && oc == 64;
    }
    m->stats = st;
}

bool build_model(AexrtYoloModel* m) {
    if (!infer_dims(m)) return false;
    fuse_residuals(m);
    Engine& e = m->eng;
    // kernel resolution (before placement: the input layout depends on it)
    for (size_t ci = 0; ci < e.commands.size(); ++ci) {
        ConvState& cs = m->convs[ci];
        if (!cs.is_conv) continue;
        const EngineCommand& c = e.commands[ci];
        const AexrtConv2DDesc d = desc_of(c);
        if (!generic_shape_ok(d))
            return fail(m, "command " + std::to_string(ci) + ": conv geometry not supported (groups/dilation)");
        cs.planned = (c.plan_flags & 1u) ? c.plan_kernel : c.planned_kernel;
        cs.algorithm = resolve_algorithm(m, ci, cs.planned);
        set_int8_mode(m, ci);
    }
    if (!plan_memory(m, m->copies)) return false;
    m->fuse_mask = 0;
    m->chain_mask = 0;
    const int fusable = fuse_head_1x1(m);
    setup_chains(m);
    // the superblocks start off; the schedule choice turns them on where faster
    m->superblock_mask = 0;
    setup_pairs(m);
    mark_slot_readers(m);
    // arena
    size_t total = 0;
    for (Root& r : m->roots) {
        r.byte_offset = total;
        total += (size_t(r.elements) * (r.f32 ? 4 : 2) + 255) & ~size_t(255);
    }
    m->arena = static_cast<uint8_t*>(dev_alloc(m, total));
    // kSlotStripes copies of the slot array, 4 KB apart
    m->slot_stride = (uint32_t)((m->nslots + 1 + 1023) & ~1023);
    m->slots = static_cast<uint32_t*>(dev_alloc(m, size_t(kSlotStripes) * m->slot_stride * 4));
    const ValueInfo& in = m->vals[e.manifest.input_value];
    const size_t in_elems = size_t(in.N) * in.C * in.H * in.W;
    m->input_dev = static_cast<float*>(dev_alloc(m, in_elems * 4));
    if (!m->arena || !m->slots || !m->input_dev) return fail(m, "out of device memory for activations");
    if (hipHostMalloc(reinterpret_cast<void**>(&m->input_host), in_elems * 4, hipHostMallocDefault) != hipSuccess)
        m->input_host = nullptr;
    for (size_t ci = 0; ci < e.commands.size(); ++ci)
        if (m->convs[ci].is_conv && !prepare_conv_weights(m, ci)) return false;
    for (size_t ci = 0; ci < e.commands.size(); ++ci)
        if (m->sibling[ci] >= 0 && !pair_conv_weights(m, ci)) return false;
    if (!check_hip(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "stream create"))
        return fail(m, last_error());
    for (int l = 1; l < kLanes; ++l)
        if (!check_hip(hipStreamCreateWithFlags(&m->lane_stream[l], hipStreamNonBlocking), "lane stream create"))
            return fail(m, last_error());
    const char* tune = std::getenv("AEXRT_HIP_AUTOTUNE");
    m->autotune = !(tune && tune[0] == '0');
    const char* tlog = std::getenv("AEXRT_HIP_TUNE_LOG");
    m->tune_log = tlog && tlog[0] == '1';
    // AEXRT_HIP_TUNE_CACHE=<file>: choices measured by an earlier load are
    // reused (and, when measuring, the file is rewritten with this load's); with
    // AEXRT_HIP_AUTOTUNE=0 the cached choices still apply, nothing is measured
    // and the file is left as it is
    const char* tcache = std::getenv("AEXRT_HIP_TUNE_CACHE");
    if (tcache && tcache[0]) {
        m->tune_cache = tcache;
        load_tune_cache(m);
    }
    // AEXRT_HIP_LANES=<n>: fixed number of streams for the captured schedule
    // (1 = steps in launch order, e.g. for a per-kernel trace); otherwise the
    // fastest lane count from kLanes down to 1, measured.  Sibling convs run as one launch or as
    // two (which can overlap on separate lanes): with pairs in the plan, both
    // schedules are measured and the faster kept.
    const char* lanes = std::getenv("AEXRT_HIP_LANES");
    const bool fixed_lanes = lanes && lanes[0] >= '1' && lanes[0] <= '9';
    // AEXRT_HIP_LIST_SCHEDULE=0 / 1: steps put on lanes by the dependency rule / by
    // list scheduling over their measured times; otherwise both are measured (with
    // autotuning) or the cached lane plan is taken
    const char* ls = std::getenv("AEXRT_HIP_LIST_SCHEDULE");
    m->lane_policy_forced = ls && (ls[0] == '0' || ls[0] == '1') ? ls[0] - '0' : -1;
    const int fixed_policy = std::max(0, m->lane_policy_forced);
    const bool pairs = std::any_of(m->sibling.begin(), m->sibling.end(), [](int s) { return s >= 0; });
    // AEXRT_HIP_FUSE_1X1=0 / 1: head 3x3 + 1x1 pairs never / always in one launch; otherwise
    // both are measured (with autotuning) or the cached schedule's choice is taken
    const char* f1 = std::getenv("AEXRT_HIP_FUSE_1X1");
    const int fuse_forced = f1 && (f1[0] == '0' || f1[0] == '1') ? f1[0] - '0' : -1;
    // AEXRT_HIP_CHAIN=0 / 1: head branches (3x3, 3x3, 1x1) never / always in one
    // launch; otherwise measured per head level (with autotuning) or cached
    const char* ch = std::getenv("AEXRT_HIP_CHAIN");
    const int chain_forced = ch && (ch[0] == '0' || ch[0] == '1') ? ch[0] - '0' : -1;
    const bool chain_choice = !m->chains.empty() && chain_forced < 0 && m->autotune && m->use_graph;
    const bool fuse_choice = fusable > 0 && fuse_forced < 0 && m->autotune && m->use_graph;
    const int merge_variants = pairs && m->autotune && m->use_graph ? 2 : 1;
    const int variants = merge_variants * (fuse_choice ? 2 : 1);
    // without measurement, a schedule cached for this network (same input and
    // command count) is reused
    const ValueInfo& xin = m->vals[e.manifest.input_value];
    const std::string skey = "schedule " + std::to_string(xin.N) + "x" + std::to_string(xin.C) + "x" +
                             std::to_string(xin.H) + "x" + std::to_string(xin.W) + " commands " +
                             std::to_string(e.commands.size());
    const auto cached_sched = m->schedules.find(skey);
    const bool use_cached_sched = !m->autotune && cached_sched != m->schedules.end();
    float best_ms = 0.0f;
    bool best_merge = true;
    uint32_t best_fuse = 0;
    int best_lanes = 1, best_policy = 0;
    // the schedule cache keeps (merge, lanes, fuse, fused pairs) in a choice's
    // (kind, jn, pw, ksw)
    auto fuse_for = [&](int k) -> uint32_t {
        if (fuse_forced >= 0) return fuse_forced ? ~0u : 0u;
        if (use_cached_sched) return schedule_fuse_mask(cached_sched->second);
        return fuse_choice && k / merge_variants == 0 ? ~0u : 0u;
    };
    // head branches while the schedule variants are measured: forced, cached
    // or none (measured afterwards)
    const uint32_t chains0 = chain_forced >= 0 ? (chain_forced ? ~0u : 0u)
                             : use_cached_sched ? cached_sched->second.chains
                                                : 0u;
    m->chain_dual = chain_forced >= 0 ? (chain_forced ? ~0u : 0u) : use_cached_sched ? cached_sched->second.dual : 0u;
    // per head pair and merge setting: the fused step's time (index 1), the
    // unfused 3x3 and 1x1 steps' (index 0)
    std::vector<float> pair_ms[2][2];
    for (int k = 0; k < variants; ++k) {
        m->merge_siblings = use_cached_sched ? cached_sched->second.first != 0 : k % merge_variants == 0;
        m->fuse_mask = fuse_for(k);
        fuse_head_1x1(m);
        m->chain_mask = chains0;
        setup_chains(m);
        m->n_lanes = 1;
        if (!build_steps(m, m->copies)) return false;
        if (m->autotune && !refine_in_context(m)) return false;
        if (fuse_choice && !pair_step_times(m, pair_ms[m->merge_siblings][m->fuse_mask ? 1 : 0])) return false;
        float ms = 0.0f;
        if (fixed_lanes) {
            m->n_lanes = std::min(kLanes, std::atoi(lanes));
            m->lane_policy = fixed_policy;
            if (!reschedule(m)) return false;
            if (variants > 1 && !time_schedule(m, &ms)) return false;
        } else if (m->autotune && !choose_lanes(m, &ms)) {
            return false;
        }
        if (k == 0 || ms < best_ms) {
            best_ms = ms;
            best_merge = m->merge_siblings;
            best_fuse = m->fuse_mask;
            best_lanes = m->n_lanes;
            best_policy = m->lane_policy;
        }
    }
    // each pair fused or not by its own step times (one launch against two,
    // under the chosen merge setting); a mixed choice takes its lane count anew
    bool mixed = false;
    if (fuse_choice) {
        const std::vector<float>& f = pair_ms[best_merge][1];
        const std::vector<float>& u = pair_ms[best_merge][0];
        uint32_t mask = 0, all = 0;
        for (size_t q = 0; q < m->fuse_pairs.size() && q < 32; ++q) {
            all |= 1u << q;
            if (q < f.size() && q < u.size() && f[q] <= u[q]) mask |= 1u << q;
        }
        mask = mask == all ? ~0u : mask;
        mixed = mask != 0u && mask != ~0u;
        best_fuse = mask;
    }
    if (best_merge != m->merge_siblings || best_fuse != m->fuse_mask) {
        // the choices of this build were measured with the variants: cached in m->refined
        m->merge_siblings = best_merge;
        m->fuse_mask = best_fuse;
        fuse_head_1x1(m);
        setup_chains(m);
        m->n_lanes = 1;
        if (!build_steps(m, m->copies)) return false;
        if (m->autotune && !refine_in_context(m)) return false;
        float ms = 0.0f;
        if (mixed && !fixed_lanes && m->autotune) {
            if (!choose_lanes(m, &ms)) return false;
        } else {
            m->n_lanes = fixed_lanes ? std::min(kLanes, std::atoi(lanes)) : best_lanes;
            m->lane_policy = fixed_lanes ? fixed_policy : best_policy;
            if (!reschedule(m)) return false;
        }
        drop_graph(m);
    }
    // the lane plan of a list-scheduled network is kept beside its schedule
    const std::string lkey = "lanes" + skey.substr(8);
    if (use_cached_sched && !fixed_lanes) {
        m->n_lanes = std::max(1, std::min(kLanes, cached_sched->second.second));
        const auto plan = m->lane_plans.find(lkey);
        m->lane_policy = m->lane_policy_forced >= 0 ? m->lane_policy_forced : plan != m->lane_plans.end() ? 2 : 0;
        m->lane_plan = plan != m->lane_plans.end() ? plan->second : std::string();
        if (!reschedule(m)) return false;
    }
    // head branches on the chain kernel, per head level (the branches reading
    // one input): the captured schedule timed with the level's branches as a
    // launch each and as one launch together, against the current steps; the
    // fastest kept
    if (chain_choice) {
        auto rebuild = [&]() {
            const int lanes_kept = m->n_lanes;
            fuse_head_1x1(m);
            setup_chains(m);
            m->n_lanes = 1;
            if (!build_steps(m, m->copies)) return false;
            if (!refine_in_context(m)) return false;
            m->n_lanes = lanes_kept;
            return reschedule(m);
        };
        float base = 0.0f;
        if (!time_schedule(m, &base)) return false;
        std::vector<uint32_t> levels;  // input value of each level, in command order
        for (const auto& c3 : m->chains) {
            const uint32_t in = e.commands[c3[0]].inputs[0];
            if (std::find(levels.begin(), levels.end(), in) == levels.end()) levels.push_back(in);
        }
        for (uint32_t lv : levels) {
            uint32_t bits = 0;
            for (size_t k = 0; k < m->chains.size() && k < 32; ++k)
                if (e.commands[m->chains[k][0]].inputs[0] == lv) bits |= 1u << k;
            // the level's branches one launch each (side by side on the lanes), then
            // both in one launch
            const uint32_t kept = m->chain_mask, kept_dual = m->chain_dual;
            uint32_t best_mask = kept, best_dual = kept_dual;
            for (int variant = 0; variant < 2; ++variant) {
                m->chain_mask = kept | bits;
                m->chain_dual = variant ? (kept_dual | bits) : (kept_dual & ~bits);
                if (!rebuild()) return false;
                float ms = 0.0f;
                if (!time_schedule(m, &ms)) return false;
                const bool faster = ms < base * 0.995f;
                if (m->tune_log)
                    std::fprintf(stderr, "aexrt head branches on value %u %s: %.1f us against %.1f us%s\n", lv,
                                 variant ? "in one launch" : "one launch each", ms * 100.0f, base * 100.0f,
                                 faster ? " (kept)" : "");
                if (faster) {
                    base = ms;
                    best_mask = m->chain_mask;
                    best_dual = m->chain_dual;
                }
            }
            if (best_mask != m->chain_mask || best_dual != m->chain_dual) {
                m->chain_mask = best_mask;
                m->chain_dual = best_dual;
                if (!rebuild()) return false;
            }
        }
    }
    // C2f bottleneck superblocks (AEXRT_HIP_C2F_SUPERBLOCK=0 / 1: never / always):
    // per arithmetic, the captured schedule timed with its pairs as superblocks
    // against the current steps, the faster kept; without measurement the cached
    // schedule's choice
    {
        const char* sb = std::getenv("AEXRT_HIP_C2F_SUPERBLOCK");
        const int sb_forced = sb && (sb[0] == '0' || sb[0] == '1') ? sb[0] - '0' : -1;
        m->superblock_mask = 3u;
        const uint32_t avail = (uint32_t)setup_pairs(m);
        m->superblock_mask = 0;
        setup_pairs(m);
        uint32_t want = 0;
        if (sb_forced >= 0) want = sb_forced ? avail : 0u;
        else if (use_cached_sched) want = (uint32_t)cached_sched->second.super & avail;
        auto rebuild_pairs = [&]() {
            const int lanes_kept = m->n_lanes;
            setup_pairs(m);
            m->n_lanes = 1;
            if (!build_steps(m, m->copies)) return false;
            if (m->autotune && !refine_in_context(m)) return false;
            m->n_lanes = lanes_kept;
            return reschedule(m);
        };
        if (sb_forced < 0 && !use_cached_sched && avail && m->autotune && m->use_graph) {
            float base = 0.0f;
            if (!time_schedule(m, &base)) return false;
            for (uint32_t bit : {1u, 2u}) {
                if (!(avail & bit)) continue;
                m->superblock_mask = want | bit;
                if (!rebuild_pairs()) return false;
                float ms = 0.0f;
                if (!time_schedule(m, &ms)) return false;
                const bool faster = ms < base * 0.995f;
                if (m->tune_log)
                    std::fprintf(stderr, "aexrt %s C2f superblocks: %.1f us against %.1f us%s\n",
                                 bit == 1u ? "fp16" : "int8", ms * 100.0f, base * 100.0f, faster ? " (kept)" : "");
                if (faster) {
                    want |= bit;
                    base = ms;
                }
            }
        }
        if (m->superblock_mask != want) {
            m->superblock_mask = want;
            if (!rebuild_pairs()) return false;
        }
    }
    // the lanes measured again over the final steps (the branches and
    // superblocks chosen above change them)
    float final_ms = 0.0f;
    if (m->autotune && !fixed_lanes && !choose_lanes(m, &final_ms)) return false;
    if (m->autotune) {
        m->schedules[skey] = Schedule{m->merge_siblings ? 1 : 0, m->n_lanes, m->fuse_mask ? 1 : 0,
                                      m->fuse_mask == ~0u ? 0u : m->fuse_mask, m->chain_mask, m->chain_dual,
                                      (int)m->superblock_mask};
        if (m->lane_policy == 1 && m->n_lanes > 1)
            m->lane_plans[lkey] = lane_digits(m);
        else
            m->lane_plans.erase(lkey);
    }
    if (m->tune_log && variants > 1)
        std::fprintf(stderr, "aexrt sibling convs: %s, head 1x1 convs fused: %s (mask %#x)\n",
                     best_merge ? "one launch" : "two launches",
                     best_fuse == ~0u ? "all" : best_fuse ? "some" : "none", best_fuse);
    if (m->autotune && !m->tune_cache.empty()) save_tune_cache(m);
    const char* prof = std::getenv("AEXRT_HIP_PROFILE");
    m->profile = prof && prof[0] == '1';
    setup_postprocess(m);
    label_steps(m);
    compute_stats(m);
    if (m->tune_log)
        for (size_t i = 0; i < m->steps.size(); ++i) {
            std::string deps;
            for (int d : m->steps[i].deps) deps += " " + std::to_string(d);
            std::fprintf(stderr, "aexrt step %zu lane %d%s after%s: %s\n", i, m->steps[i].lane,
                         m->steps[i].signal ? " signals" : "", deps.c_str(), m->steps[i].label.c_str());
        }
    m->executable = true;
    return true;
}

void free_model(AexrtYoloModel* m) {
    if (!m) return;
    // teardown: errors are not actionable here, every resource is released anyway
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    drop_graph(m);
    for (void* p : m->allocations) (void)hipFree(p);
    if (m->input_host) (void)hipHostFree(m->input_host);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    for (int l = 1; l < kLanes; ++l)
        if (m->lane_stream[l]) (void)hipStreamDestroy(m->lane_stream[l]);
    for (hipEvent_t e : m->step_events)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : m->lane_events)
        if (e) (void)hipEventDestroy(e);
    delete m;
}

AexrtYoloModel* load_from_bytes(AexrtDevice* device, const uint8_t* data, size_t n) {
    if (!device) {
        set_error("load_engine: null device");
        return nullptr;
    }
    AexrtYoloModel* m = new AexrtYoloModel();
    m->device = device;
    std::string err;
    if (!parse_engine(data, n, m->eng, err) || !expand_fused_commands(m->eng, err)) {
        set_error(err);
        free_model(m);
        return nullptr;
    }
    if (hipSetDevice(device->index) != hipSuccess) {
        set_error("load_engine: cannot select device");
        free_model(m);
        return nullptr;
    }
    if (!build_model(m)) {
        set_error(m->last_error);
        free_model(m);
        return nullptr;
    }
    return m;
}

bool copy_value_to_host(AexrtYoloModel* m, int v, float* out, uint64_t elements) {
    const ValueInfo& x = m->vals[v];
    if (!x.pl.valid) return fail(m, "value has no device storage");
    const uint64_t n = uint64_t(x.N) * x.C * x.H * x.W;
    if (elements < n) return fail(m, "output buffer too small");
    float* tmp = nullptr;
    if (hipMalloc(&tmp, n * 4) != hipSuccess) return fail(m, "out of device memory");
    AexrtHipTensorView tv = view_of(m, v);
    hipError_t e = launch_nhwc_to_nchw_f32(tv.data, !is_f32(m, v), tv.n_stride, tv.c_stride, tmp, x.N, x.C,
                                           x.H * x.W, m->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, tmp, n * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    const hipError_t ef = hipFree(tmp);
    if (e == hipSuccess) e = ef;
    if (e != hipSuccess) return fail(m, std::string("readback: ") + hipGetErrorString(e));
    return true;
}

uint32_t conv_candidates(AexrtYoloModel* m, size_t ci, uint32_t* ids, uint32_t cap) {
    const EngineCommand& c = m->eng.commands[ci];
    const AexrtConv2DDesc d = desc_of(c);
    uint32_t n = 0;
    auto push = [&](uint32_t id) {
        if (n < cap) ids[n++] = id;
    };
    push(5);
    const ValueInfo& x = m->vals[c.inputs[0]];
    // an NHWC copy of the network input exists only when the plan needs one
    const bool nhwc_input = !x.is_input || m->input_needs_nhwc;
    if (winograd_shape_ok(d) && c.kind == kCmdConvSilu && nhwc_input) push(40);
    if (nhwc_input) {
        if (d.kernel_h == 1 && can_use_int8(d, 1)) push(51);
        if (d.kernel_h == 3 && d.stride_h == 1 && can_use_int8(d, 9)) push(52);
        if (d.kernel_h == 3 && d.stride_h == 2 && can_use_int8(d, 9)) push(53);
    }
    return n;
}

}  // namespace
}  // namespace aexrt

extern "C" {

AexrtDevice* aexrt_hip_create_device(uint32_t device_index) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || (int)device_index >= count) {
        set_error("create_device: no such HIP device");
        return nullptr;
    }
    AexrtDevice* d = new AexrtDevice();
    d->index = (int)device_index;
    if (hipGetDeviceProperties(&d->props, d->index) != hipSuccess || hipSetDevice(d->index) != hipSuccess) {
        delete d;
        set_error("create_device: cannot query device");
        return nullptr;
    }
    return d;
}

void aexrt_hip_destroy_device(AexrtDevice* device) { delete device; }

// The reference's device entry points (native/aexrt.h:129-140) under their
// own names, so that its ctypes binding loads this library unchanged.
int aexrt_d3d12_probe(void) {
    int count = 0;
    return hipGetDeviceCount(&count) == hipSuccess && count > 0 ? 1 : 0;
}
AexrtDevice* aexrt_d3d12_create_device(uint32_t adapter_index) { return aexrt_hip_create_device(adapter_index); }
void aexrt_d3d12_destroy_device(AexrtDevice* device) { aexrt_hip_destroy_device(device); }
int aexrt_d3d12_get_capabilities(AexrtDevice* device, AexrtD3D12Capabilities* caps) {
    if (!device || !caps || caps->struct_size < sizeof(AexrtD3D12Capabilities)) {
        set_error("get_capabilities: bad arguments");
        return 0;
    }
    const bool gfx950 = std::strncmp(device->props.gcnArchName, "gfx950", 6) == 0;
    caps->struct_size = sizeof(AexrtD3D12Capabilities);
    caps->highest_shader_model = 0;  // no D3D shader model: HIP code objects
    caps->native_fp16_supported = 1;
    caps->wave_mma_tier = gfx950 ? 1u : 0u;  // matrix cores (MFMA)
    caps->dxc_available = 0;
    caps->reserved[0] = caps->reserved[1] = caps->reserved[2] = 0;
    return 1;
}

// Building from an ONNX file or a package directory is the compiler's job
// (aexrt_amd.engine writes the .aexrt engine); the runtime loads engines.
AexrtYoloModel* aexrt_yolo_compile_from_package(AexrtDevice* device, const char* package_path) {
    (void)device, (void)package_path;
    set_error("compile_from_package: not supported; build a .aexrt engine and call aexrt_yolo_load_engine");
    return nullptr;
}
AexrtYoloModel* aexrt_yolo_compile_from_onnx(AexrtDevice* device, const char* onnx_path) {
    (void)device, (void)onnx_path;
    set_error("compile_from_onnx: not supported; build a .aexrt engine and call aexrt_yolo_load_engine");
    return nullptr;
}

int aexrt_hip_get_capabilities(AexrtDevice* device, AexrtHipCapabilities* caps) {
    if (!device || !caps || caps->struct_size < sizeof(AexrtHipCapabilities)) {
        set_error("get_capabilities: bad arguments");
        return 0;
    }
    const hipDeviceProp_t& p = device->props;
    caps->device_index = (uint32_t)device->index;
    caps->compute_units = (uint32_t)p.multiProcessorCount;
    caps->wavefront_size = (uint32_t)p.warpSize;
    caps->lds_bytes_per_block = (uint32_t)p.sharedMemPerBlock;
    const bool gfx950 = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
    caps->int8_mfma = gfx950 ? 1u : 0u;
    caps->fp16_mfma = gfx950 ? 1u : 0u;
    caps->global_mem_bytes = (uint64_t)p.totalGlobalMem;
    std::snprintf(caps->arch_name, sizeof(caps->arch_name), "%s", p.gcnArchName);
    return 1;
}

int aexrt_hip_validate_engine(const void* data, uint64_t nbytes) {
    if (!data) {
        set_error("validate_engine: null data");
        return 0;
    }
    // the container rules, then the shape inference of the load (host only)
    AexrtYoloModel m;
    std::string err;
    if (!parse_engine(static_cast<const uint8_t*>(data), (size_t)nbytes, m.eng, err) ||
        !expand_fused_commands(m.eng, err)) {
        set_error(err);
        return 0;
    }
    return infer_dims(&m) ? 1 : 0;
}

AexrtYoloModel* aexrt_yolo_load_engine_memory(AexrtDevice* device, const void* data, uint64_t nbytes) {
    if (!data) {
        set_error("load_engine_memory: null data");
        return nullptr;
    }
    return load_from_bytes(device, static_cast<const uint8_t*>(data), (size_t)nbytes);
}

AexrtYoloModel* aexrt_yolo_load_engine(AexrtDevice* device, const char* engine_path) {
    if (!engine_path) {
        set_error("load_engine: null path");
        return nullptr;
    }
    std::ifstream f(engine_path, std::ios::binary);
    if (!f) {
        set_error(std::string("load_engine: cannot open ") + engine_path);
        return nullptr;
    }
    std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    return load_from_bytes(device, bytes.data(), bytes.size());
}

uint64_t aexrt_yolo_input_element_count(AexrtYoloModel* m) {
    if (!m) return 0;
    const auto& x = m->vals[m->eng.manifest.input_value];
    return uint64_t(x.N) * x.C * x.H * x.W;
}

uint64_t aexrt_yolo_output_element_count(AexrtYoloModel* m) {
    if (!m) return 0;
    const auto& x = m->vals[m->eng.manifest.output_value];
    return uint64_t(x.N) * x.C * x.H * x.W;
}

uint32_t aexrt_yolo_class_count(AexrtYoloModel* m) { return m ? m->eng.manifest.classes : 0; }
uint32_t aexrt_yolo_anchor_count(AexrtYoloModel* m) { return m ? m->eng.manifest.anchors : 0; }
uint32_t aexrt_yolo_channel_count(AexrtYoloModel* m) { return m ? m->eng.manifest.channels : 0; }
uint32_t aexrt_yolo_output_layout(AexrtYoloModel* m) { return m ? m->eng.manifest.layout : 0; }
uint32_t aexrt_yolo_has_objectness(AexrtYoloModel* m) { return m ? m->eng.manifest.has_objectness : 0; }
uint32_t aexrt_yolo_graph_node_count(AexrtYoloModel* m) { return m ? m->eng.manifest.graph_node_count : 0; }
uint32_t aexrt_yolo_graph_value_count(AexrtYoloModel* m) { return m ? (uint32_t)m->eng.values.size() : 0; }
uint32_t aexrt_yolo_constant_count(AexrtYoloModel* m) { return m ? m->eng.manifest.constant_count : 0; }
uint32_t aexrt_yolo_prepared_command_count(AexrtYoloModel* m) { return m ? m->eng.manifest.command_count : 0; }
int aexrt_yolo_is_executable(AexrtYoloModel* m) { return m && m->executable ? 1 : 0; }

// A model loaded from an .aexrt engine is a native graph with the YOLO
// postprocess (AEXRT_YOLO_PACKAGE_NATIVE_D3D12_GRAPH, native/aexrt.h:53-57).
uint32_t aexrt_yolo_package_mode(AexrtYoloModel* m) { return m ? 2u : 0u; }
// Every command of an accepted engine runs (the loader refuses the others).
uint32_t aexrt_yolo_supported_prepared_command_count(AexrtYoloModel* m) { return m ? m->eng.manifest.command_count : 0; }
uint32_t aexrt_yolo_unsupported_prepared_command_count(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_prepared_skipped_command_count(AexrtYoloModel* m) { return m ? m->stats.skipped : 0; }
uint32_t aexrt_yolo_late_concat_conv1x1_fusion_count(AexrtYoloModel* m) { return m ? m->stats.late_concat_conv1x1 : 0; }
// D3D12-only fusions this backend does not form: 0.
uint32_t aexrt_yolo_concat_residual_conv1x1_fusion_count(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_paired_conv3x3_fusion_count(AexrtYoloModel* m) { return m ? m->stats.paired_conv3x3 : 0; }
uint32_t aexrt_yolo_c2f_bottleneck_superblock_count(AexrtYoloModel* m) { return m ? m->stats.c2f_superblocks : 0; }
uint32_t aexrt_yolo_c2f_tail_residual_fusion_count(AexrtYoloModel* m) { return m ? m->stats.tail_residual : 0; }
uint32_t aexrt_yolo_head_fusion_enabled(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_head_final_conv_fusion_enabled(AexrtYoloModel* m) { return m && m->stats.head_final_conv ? 1u : 0u; }
uint32_t aexrt_yolo_tileflow_conv1x1_count(AexrtYoloModel* m) { return m ? m->stats.conv1x1 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_spatial_count(AexrtYoloModel* m) { return m ? m->stats.spatial3x3 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_pack4_count(AexrtYoloModel* m) { return m ? m->stats.pack4_3x3 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_pack8_count(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_count(AexrtYoloModel* m) { return m ? m->stats.igemm3x3 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_40x40_count(AexrtYoloModel* m) { return m ? m->stats.igemm3x3_40 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_20x20_count(AexrtYoloModel* m) { return m ? m->stats.igemm3x3_20 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_implicit_gemm_10x10_count(AexrtYoloModel* m) { return m ? m->stats.igemm3x3_10 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_exact_40x40_64x64_count(AexrtYoloModel* m) { return m ? m->stats.exact_40_64x64 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_exact_20x20_64x64_count(AexrtYoloModel* m) { return m ? m->stats.exact_20_64x64 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_exact_10x10_128x128_count(AexrtYoloModel* m) { return m ? m->stats.exact_10_128x128 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_exact_20x20_128x64_count(AexrtYoloModel* m) { return m ? m->stats.exact_20_128x64 : 0; }
uint32_t aexrt_yolo_tileflow_3x3_exact_10x10_256x64_count(AexrtYoloModel* m) { return m ? m->stats.exact_10_256x64 : 0; }
uint32_t aexrt_yolo_tileflow_native_fp16_count(AexrtYoloModel* m) { return m ? m->stats.native_fp16 : 0; }

// Runs are synchronous (no frames in flight): like the reference with one
// pipeline frame (native/aexrt.h:412-416), flushing yields 0 detections.
int aexrt_yolo_flush_pipeline(AexrtYoloModel* m, AexrtYoloDetection* detections, uint32_t max_detections,
                              uint32_t* out_detection_count) {
    if (!m || !detections || !out_detection_count || max_detections == 0) return 0;
    *out_detection_count = 0;
    return 1;
}

// No shader or pipeline objects are compiled at load (the HIP code objects
// are part of the library): the exported cache is the valid empty one, a
// 16-byte header (version 1, no shader or PSO records, flags 1), as the
// reference builds it with no entries (RT:31062-31101).
uint64_t aexrt_yolo_pipeline_cache_size(AexrtYoloModel* m) { return m ? 16u : 0u; }
int aexrt_yolo_export_pipeline_cache(AexrtYoloModel* m, void* output, uint64_t output_nbytes) {
    if (!m || !output || output_nbytes < 16) return 0;
    const uint32_t header[4] = {1u, 0u, 0u, 1u};
    std::memcpy(output, header, sizeof(header));
    return 1;
}
uint32_t aexrt_yolo_dxil_cache_hit_count(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_shader_cache_hit_count(AexrtYoloModel* m) { (void)m; return 0; }
uint32_t aexrt_yolo_pso_cache_hit_count(AexrtYoloModel* m) { (void)m; return 0; }

void* aexrt_yolo_input_device_ptr(AexrtYoloModel* m) { return m ? m->input_dev : nullptr; }

void* aexrt_yolo_input_ptr(AexrtYoloModel* m, uint64_t* out_elements) {
    if (!m) return nullptr;
    if (out_elements) *out_elements = aexrt_yolo_input_element_count(m);
    return m->input_host;
}

int aexrt_yolo_run_device(AexrtYoloModel* m, const float* input, void* stream, void* reserved) {
    (void)reserved;
    if (!m || !m->executable) {
        set_error("run_device: model is not executable");
        return 0;
    }
    std::lock_guard<std::mutex> lock(m->mutex);
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->stream;
    if (input && input != m->input_dev) {
        const size_t bytes = aexrt_yolo_input_element_count(m) * 4;
        if (!check_hip(hipMemcpyAsync(m->input_dev, input, bytes, hipMemcpyDeviceToDevice, s), "input copy"))
            return fail(m, last_error()) ? 1 : 0;
    }
    return run_network(m, s) ? 1 : 0;
}

int aexrt_yolo_postprocess_device(AexrtYoloModel* m, void* stream, float** detections_device,
                                  uint32_t** count_device) {
    if (!m || !m->executable || !m->post_ok) {
        set_error("postprocess_device: the engine's output is not a YOLO head this backend decodes");
        if (m) m->last_error = "postprocess_device: no YOLO postprocess for this engine";
        return 0;
    }
    std::lock_guard<std::mutex> lock(m->mutex);
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->stream;
    if (!launch_postprocess(m, s)) return fail(m, last_error()) ? 1 : 0;
    if (detections_device) *detections_device = m->dets_dev;
    if (count_device) *count_device = m->det_count_dev;
    return 1;
}

int aexrt_yolo_run(AexrtDevice* device, AexrtYoloModel* m, const float* input, uint64_t input_element_count,
                   AexrtYoloDetection* detections, uint32_t max_detections, uint32_t* out_detection_count) {
    if (!device || !m || !input) {
        set_error("run: null argument");
        if (m) m->last_error = "run: null argument";
        return 0;
    }
    if (m->device != device) return fail(m, "run: model belongs to another device") ? 1 : 0;
    if (!m->executable) return fail(m, "run: model is not executable") ? 1 : 0;
    const uint64_t n = aexrt_yolo_input_element_count(m);
    if (input_element_count < n) return fail(m, "run: input too small") ? 1 : 0;
    std::lock_guard<std::mutex> lock(m->mutex);
    std::lock_guard<std::mutex> dlock(device->mutex);
    using clk = std::chrono::steady_clock;
    AexrtYoloRunTiming t{};
    t.struct_size = sizeof(t);
    auto t0 = clk::now();
    const float* src = input;
    if (m->input_host && input != m->input_host) {
        std::memcpy(m->input_host, input, n * 4);
        src = m->input_host;
    }
    if (!check_hip(hipMemcpyAsync(m->input_dev, src, n * 4, hipMemcpyHostToDevice, m->stream), "input upload"))
        return fail(m, last_error()) ? 1 : 0;
    auto t1 = clk::now();
    if (!run_network(m, m->stream)) return 0;
    // decode + NMS + top-k of output0 on the device (RT:27104-27219), then
    // the reference's readback: count = min(device count, caller capacity,
    // the engine's max_detections) (RT:29699-29728)
    uint32_t raw_count = 0;
    std::vector<float> dets_host;
    if (m->post_ok) {
        dets_host.resize(size_t(m->eng.manifest.max_detections) * 6);
        if (!launch_postprocess(m, m->stream) ||
            !check_hip(hipMemcpyAsync(&raw_count, m->det_count_dev, 4, hipMemcpyDeviceToHost, m->stream),
                       "detection count readback") ||
            !check_hip(hipMemcpyAsync(dets_host.data(), m->dets_dev, dets_host.size() * 4, hipMemcpyDeviceToHost,
                                      m->stream),
                       "detection readback")) {
            // a readback already enqueued writes into raw_count / dets_host: it
            // completes before they go out of scope
            const std::string err = last_error();
            (void)hipStreamSynchronize(m->stream);
            return fail(m, err) ? 1 : 0;
        }
    }
    auto t2 = clk::now();
    if (!check_hip(hipStreamSynchronize(m->stream), "run sync")) return fail(m, last_error()) ? 1 : 0;
    if (m->pair_err) {  // a superblock's grid barrier wait that timed out leaves wrong outputs
        uint32_t err = 0;
        if (!check_hip(hipMemcpy(&err, m->pair_err, 4, hipMemcpyDeviceToHost), "superblock status") || err)
            return fail(m, err ? "run: a C2f superblock's grid barrier timed out (the outputs are not valid)"
                               : last_error()) ? 1 : 0;
    }
    auto t3 = clk::now();
    uint32_t cap = 0;
    if (m->post_ok && detections)
        cap = std::min({raw_count, max_detections, m->eng.manifest.max_detections});
    if (cap) std::memcpy(detections, dets_host.data(), size_t(cap) * sizeof(AexrtYoloDetection));
    if (out_detection_count) *out_detection_count = cap;
    auto t4 = clk::now();
    auto ms = [](clk::time_point a, clk::time_point b) {
        return std::chrono::duration<double, std::milli>(b - a).count();
    };
    t.valid = 1;
    t.memcpy_ms = ms(t0, t1);
    t.submit_ms = ms(t1, t2);
    t.fence_ms = ms(t2, t3);
    t.readback_ms = ms(t3, t4);
    m->timing = t;
    return 1;
}

int aexrt_yolo_debug_output(AexrtYoloModel* m, float* out, uint64_t elements) {
    if (!m || !out) return 0;
    std::lock_guard<std::mutex> lock(m->mutex);
    if (!check_hip(hipStreamSynchronize(m->stream), "debug output sync")) return fail(m, last_error()) ? 1 : 0;
    return copy_value_to_host(m, (int)m->eng.manifest.output_value, out, elements) ? 1 : 0;
}

int aexrt_yolo_debug_value(AexrtYoloModel* m, uint32_t value_id, float* out, uint64_t elements) {
    if (!m || !out || value_id >= m->vals.size()) return 0;
    std::lock_guard<std::mutex> lock(m->mutex);
    if (!check_hip(hipStreamSynchronize(m->stream), "debug value sync")) return fail(m, last_error()) ? 1 : 0;
    int v = (int)value_id;
    if (m->vals[v].redirect >= 0) return fail(m, "value was fused into a residual add and is never stored") ? 1 : 0;
    if (m->vals[v].is_input) {
        const uint64_t n = aexrt_yolo_input_element_count(m);
        if (elements < n) return 0;
        return hipMemcpy(out, m->input_dev, n * 4, hipMemcpyDeviceToHost) == hipSuccess ? 1 : 0;
    }
    // upsamples that the convs reading them take from their sources are stored now
    if (m->vals[v].pl.valid && !store_folded_upsamples(m, m->vals[v].pl.root)) return fail(m, last_error()) ? 1 : 0;
    return copy_value_to_host(m, v, out, elements) ? 1 : 0;
}

int aexrt_yolo_debug_conv_int8(AexrtYoloModel* m, uint32_t command_index, int32_t* acc, uint64_t acc_elements,
                               uint32_t* slots, uint32_t slot_count) {
    if (!m || !acc) return 0;
    std::lock_guard<std::mutex> lock(m->mutex);
    const Step* st = nullptr;
    for (const Step& s : m->steps)
        if (s.cmd >= 0 && s.conv_params && m->eng.src_cmd[s.cmd] == command_index) st = &s;
    if (!st) return fail(m, "debug_conv_int8: command " + std::to_string(command_index) +
                                " is not a per-tensor int8 conv of the prepared steps") ? 1 : 0;
    ConvParams q = st->conv_params();
    const uint64_t n_acc = (uint64_t)q.M * (uint64_t)q.OC;
    if (acc_elements < n_acc || (slots && slot_count < (uint32_t)q.x_nslots))
        return fail(m, "debug_conv_int8: output buffers too small") ? 1 : 0;
    if (!check_hip(hipStreamSynchronize(m->stream), "debug_conv_int8 sync")) return fail(m, last_error()) ? 1 : 0;
    // the conv again on the input the last run left in memory, with the same
    // kernel and tile: accumulators on, its output into a dense scratch view,
    // no amax slot updates (the model's memory is left as the run left it)
    const int esz = (q.flags & kConvOutF32) ? 4 : 2;
    void *acc_dev = nullptr, *y_dev = nullptr;
    bool ok = check_hip(hipMalloc(&acc_dev, n_acc * 4), "debug_conv_int8 alloc") &&
              check_hip(hipMalloc(&y_dev, n_acc * esz), "debug_conv_int8 alloc");
    if (ok) {
        q.acc_out = static_cast<int32_t*>(acc_dev);
        q.y = y_dev;
        q.y_nstride = (int64_t)q.OH * q.OW * q.OC;
        q.y_cstride = q.OC;
        q.y_slots = SlotRef{nullptr, 1u, 0u};
        ok = check_hip(launch_conv_igemm(q, true, m->stream), "debug_conv_int8 launch") &&
             check_hip(hipStreamSynchronize(m->stream), "debug_conv_int8 sync") &&
             check_hip(hipMemcpy(acc, acc_dev, n_acc * 4, hipMemcpyDeviceToHost), "debug_conv_int8 copy");
    }
    // the input's slot words, max over the stripes (what the conv quantized with)
    if (ok && slots) {
        const uint32_t stripes = q.x_slots.stripes ? q.x_slots.stripes : 1u;
        std::vector<uint32_t> w((size_t)q.x_nslots);
        for (uint32_t g = 0; g < (uint32_t)q.x_nslots; ++g) slots[g] = 0u;
        for (uint32_t s = 0; s < stripes && ok; ++s) {
            ok = check_hip(hipMemcpy(w.data(), q.x_slots.p + (size_t)s * q.x_slots.stride, w.size() * 4,
                                     hipMemcpyDeviceToHost),
                           "debug_conv_int8 slots");
            for (size_t g = 0; ok && g < w.size(); ++g) slots[g] = std::max(slots[g], w[g]);
        }
        // groups read from an upsampled source: its slot words
        if (ok && q.xup) {
            const uint32_t us = q.xup_slots.stripes ? q.xup_slots.stripes : 1u;
            std::vector<uint32_t> u((size_t)q.xup_nslots);
            const int g0 = q.xup_c0 / 16;
            for (uint32_t s = 0; s < us && ok; ++s) {
                ok = check_hip(hipMemcpy(u.data(), q.xup_slots.p + (size_t)s * q.xup_slots.stride, u.size() * 4,
                                         hipMemcpyDeviceToHost),
                               "debug_conv_int8 source slots");
                for (size_t g = 0; ok && g < u.size(); ++g) slots[g0 + g] = std::max(slots[g0 + g], u[g]);
            }
        }
    }
    if (acc_dev) (void)hipFree(acc_dev);
    if (y_dev) (void)hipFree(y_dev);
    if (!ok) return fail(m, last_error()) ? 1 : 0;
    return 1;
}

// The reference reads back a D3D12 arena page (native/aexrt.h:403); values
// here live in roots of one NHWC arena, read through aexrt_yolo_debug_value.
int aexrt_yolo_debug_page(AexrtYoloModel* m, uint32_t page_id, float* out, uint64_t elements) {
    (void)page_id, (void)out, (void)elements;
    if (m) m->last_error = "debug_page: no arena pages in this runtime; use aexrt_yolo_debug_value";
    set_error("debug_page: no arena pages in this runtime; use aexrt_yolo_debug_value");
    return 0;
}

int aexrt_yolo_value_info(AexrtYoloModel* m, uint32_t value_id, uint32_t* out4) {
    if (!m || !out4 || value_id >= m->vals.size()) return 0;
    const auto& x = m->vals[value_id];
    out4[0] = (uint32_t)x.N;
    out4[1] = (uint32_t)x.C;
    out4[2] = (uint32_t)x.H;
    out4[3] = (uint32_t)x.W;
    if (x.is_const || x.redirect >= 0 || x.elided || !(x.pl.valid || x.is_input)) return 0;
    return x.rank;
}

const char* aexrt_yolo_get_last_error(AexrtYoloModel* m) { return m ? m->last_error.c_str() : last_error(); }

int aexrt_yolo_get_last_run_timing(AexrtYoloModel* m, AexrtYoloRunTiming* timing) {
    if (!m || !timing || timing->struct_size < sizeof(AexrtYoloRunTiming)) return 0;
    *timing = m->timing;
    return 1;
}

int aexrt_yolo_set_profiling(AexrtYoloModel* m, int enabled) {
    if (!m) return 0;
    m->profile = enabled != 0;
    return 1;
}

uint32_t aexrt_yolo_profile_event_count(AexrtYoloModel* m) { return m ? (uint32_t)m->prof_ms.size() : 0; }

const char* aexrt_yolo_profile_event_label(AexrtYoloModel* m, uint32_t i) {
    return (m && i < m->prof_labels.size()) ? m->prof_labels[i].c_str() : "";
}

double aexrt_yolo_profile_event_ms(AexrtYoloModel* m, uint32_t i) {
    return (m && i < m->prof_ms.size()) ? m->prof_ms[i] : 0.0;
}

int aexrt_yolo_set_graph_capture(AexrtYoloModel* m, int enabled) {
    if (!m) return 0;
    m->use_graph = enabled != 0;
    drop_graph(m);
    return 1;
}

uint32_t aexrt_yolo_conv_plan_count(AexrtYoloModel* m) {
    if (!m) return 0;
    uint32_t n = 0;
    for (const auto& c : m->convs) n += c.is_conv ? 1u : 0u;
    return n;
}

int aexrt_yolo_conv_plan_info(AexrtYoloModel* m, uint32_t index, AexrtConvPlanInfo* out) {
    if (!m || !out || out->struct_size < sizeof(AexrtConvPlanInfo)) return 0;
    uint32_t k = 0;
    for (size_t ci = 0; ci < m->convs.size(); ++ci) {
        if (!m->convs[ci].is_conv) continue;
        if (k++ != index) continue;
        const EngineCommand& c = m->eng.commands[ci];
        out->command_index = m->eng.src_cmd[ci];
        out->kind_is_silu = c.kind == kCmdConvSilu ? 1u : 0u;
        out->desc = desc_of(c);
        out->current_algorithm = m->convs[ci].algorithm;
        out->candidate_count = conv_candidates(m, ci, out->candidates, 32);
        out->in_fusion_group = m->convs[ci].fused_residual ? 1u : 0u;
        out->planned_algorithm = m->convs[ci].planned;
        return 1;
    }
    return 0;
}

int aexrt_yolo_override_conv_algorithm(AexrtYoloModel* m, uint32_t engine_command, uint32_t algorithm_id) {
    // engine-file command index -> the conv it became (a CONCAT_CONV1X1 is a
    // concat followed by its conv)
    size_t command_index = SIZE_MAX;
    if (m)
        for (size_t ci = 0; ci < m->convs.size(); ++ci)
            if (m->eng.src_cmd[ci] == engine_command && m->convs[ci].is_conv) command_index = ci;
    if (!m || command_index == SIZE_MAX) {
        set_error("override: not a conv command");
        if (m) m->last_error = "override: not a conv command";
        return 0;
    }
    std::lock_guard<std::mutex> lock(m->mutex);
    uint32_t ids[32];
    const uint32_t n = conv_candidates(m, command_index, ids, 32);
    uint32_t kernel = algorithm_id;
    bool ok = false;
    for (uint32_t i = 0; i < n; ++i) ok |= ids[i] == algorithm_id;
    if (!ok && !is_int8_algorithm(algorithm_id) && !is_winograd_algorithm(algorithm_id) && algorithm_id <= 54) {
        kernel = algorithm_id;  // every other reference id runs on the generic fp16 kernel
        ok = true;
    }
    if (!ok) return fail(m, "override: algorithm not applicable to this command") ? 1 : 0;
    if (!check_hip(hipStreamSynchronize(m->stream), "override sync")) return fail(m, last_error()) ? 1 : 0;
    // Everything an override changes is kept so that a failure restores the
    // model as it was (weights stay allocated until the model is freed).
    const ConvState saved = m->convs[command_index];
    std::vector<std::pair<size_t, ConvState>> saved_pairs;
    for (size_t ci = 0; ci < m->sibling.size(); ++ci)
        if (m->sibling[ci] >= 0 && (ci == command_index || m->sibling[ci] == (int)command_index))
            saved_pairs.emplace_back(ci, m->convs[ci]);
    auto restore = [&](const std::string& why) {
        const std::string msg = "override: " + why;
        m->convs[command_index] = saved;
        for (const auto& [ci, cs] : saved_pairs) m->convs[ci] = cs;
        drop_graph(m);
        mark_slot_readers(m);
        if (!build_steps(m, m->copies) || (m->autotune && !refine_in_context(m))) {
            m->executable = false;
            fail(m, msg + "; the model could not be restored and is no longer executable");
            return 0;
        }
        compute_stats(m);
        fail(m, msg);
        return 0;
    };
    ConvState& cs = m->convs[command_index];
    cs.algorithm = kernel;
    set_int8_mode(m, command_index);
    if (!prepare_conv_weights(m, command_index)) return restore(m->last_error);
    // a sibling pair with this conv gets its joint weights from the new ones
    // (it runs as two launches while either conv is not an fp16 direct one)
    for (const auto& sp : saved_pairs)
        if (!pair_conv_weights(m, sp.first)) return restore(m->last_error);
    drop_graph(m);
    mark_slot_readers(m);
    // placement does not depend on the kernel choice: rebuild the launch list;
    // the other convs keep their measured choices (keyed by command, algorithm
    // and shape), and so does this one when it returns to an earlier algorithm
    if (!build_steps(m, m->copies)) return restore(m->last_error);
    if (m->autotune && !refine_in_context(m)) return restore(m->last_error);
    compute_stats(m);
    return 1;
}

void aexrt_yolo_destroy(AexrtYoloModel* m) { free_model(m); }

}  // extern "C"
