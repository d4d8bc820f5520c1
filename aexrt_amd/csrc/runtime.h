// Model runtime: parsed .aexrt engine, placement of values in device memory
// and the list of kernel launches one run consists of.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

namespace aexrt {

// ---- parsed engine (sections 1-6 of the container) ---------------------------
struct EngineManifest {
    uint32_t precision = 0, layout = 0, has_objectness = 0, channels = 0, anchors = 0, classes = 0;
    uint32_t max_candidates = 0, max_detections = 0, graph_node_count = 0, value_count = 0;
    uint32_t constant_count = 0, command_count = 0, input_value = 0, output_value = 0;
    uint64_t input_elements = 0, arena_nbytes = 0;
    float conf_threshold = 0.f, iou_threshold = 0.f;
};

// What the loader keeps of sections 7-9: the reference runtime's arena
// description (validated, not used: this runtime plans its own NHWC memory),
// the fusion groups (validated; their commands run one by one) and the
// pipeline-cache record count (D3D12 shader/PSO blobs, nothing to use here).
struct EngineExtras {
    uint32_t memory_plan_version = 0, arena_pages = 0, fusion_groups = 0, cache_records = 0;
    uint32_t physical_dispatch_plan = 0, barrier_plan = 0;
};

struct EngineValue {
    uint32_t id = 0, flags = 0;
    uint64_t elements = 0;
    uint32_t shape4[4] = {1, 1, 1, 1};
};

// Kernel-plan record flags (src/aexrt/engine.py:85-96): bit 0 authoritative,
// bit 4 int8 with per-16-input-channel activation scales (pg16).
constexpr uint32_t kPlanFlagAuthoritative = 1u;
constexpr uint32_t kPlanFlagInt8PerGroup = 16u;

struct EngineCommand {
    uint32_t kind = 0, output = 0, planned_kernel = 0, precision = 0;
    std::vector<uint32_t> inputs, params;
    // from the kernel plan section
    uint32_t plan_kernel = 0, plan_precision = 0, packed_value = UINT32_MAX, plan_flags = 0;
};

struct EngineConstant {
    uint32_t precision = 0;
    uint64_t elements = 0;
    std::vector<uint8_t> raw;  // fp32 or fp16 payload
    bool present = false;
};

struct EnginePacked {
    uint32_t layout = 0, in_channels = 0, out_channels = 0;
    uint64_t elements = 0;
    std::vector<uint8_t> data;
    bool present = false;
};

struct Engine {
    EngineManifest manifest;
    std::vector<EngineValue> values;
    std::vector<EngineCommand> commands;
    std::vector<EngineConstant> constants;  // indexed by value id
    std::vector<EnginePacked> packed;       // indexed by value id
    EngineExtras extras;
    // after expand_fused_commands: the engine-file command each command came
    // from (the conv plan API speaks in engine-file indices)
    std::vector<uint32_t> src_cmd;
};

enum CommandKind : uint32_t {
    kCmdConv = 1, kCmdConvSilu = 2, kCmdConcatConv1x1 = 3, kCmdView = 4, kCmdAlias = 5, kCmdSlice = 6,
    kCmdConcat = 7, kCmdResize = 8, kCmdMaxpool = 9, kCmdUnary = 10, kCmdBinary = 11, kCmdMatmul = 12,
    kCmdTranspose = 13, kCmdSoftmax = 14,
};

bool parse_engine(const uint8_t* data, size_t size, Engine& out, std::string& err);
// Rewrites each CONCAT_CONV1X1 command (yolo.py:771-779: inputs x0..x(k-1),
// weight, bias; params N, H, W, OC, silu, then the k input channel counts)
// into a channel CONCAT into a new value followed by a 1x1 CONV / CONV_SILU
// on it, and fills src_cmd.  The concat is then placed like every other one
// (producers write straight into its channel slices), so the fused command
// costs one 1x1 conv over the concatenated channels.
bool expand_fused_commands(Engine& e, std::string& err);
uint32_t crc32_ieee(const uint8_t* data, size_t size);

}  // namespace aexrt
