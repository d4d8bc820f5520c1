// .aexrt container parser (sections 1-6).  Every offset and size is checked
// against the buffer before it is read, every section's CRC32 is verified,
// and an engine whose plan disagrees with its packed weights is rejected
// (the loader's fail-closed rules, native/aexrt_d3d12_runtime.cpp:17560-18164).
#include <algorithm>
#include <cstring>
#include <string>

#include "runtime.h"

namespace aexrt {

namespace {

constexpr char kMagic[8] = {'A', 'E', 'X', 'R', 'T', 'E', 'N', 'G'};

template <typename T>
bool rd(const uint8_t* base, size_t size, size_t off, T& v) {
    if (off > size || size - off < sizeof(T)) return false;
    std::memcpy(&v, base + off, sizeof(T));
    return true;
}

struct Section {
    const uint8_t* data = nullptr;
    size_t size = 0;
};

}  // namespace

uint32_t crc32_ieee(const uint8_t* data, size_t size) {
    static uint32_t table[256];
    static bool init = false;
    if (!init) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
        init = true;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < size; ++i) c = table[(c ^ data[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

bool expand_fused_commands(Engine& e, std::string& err) {
    std::vector<EngineCommand> cmds;
    std::vector<uint32_t> src;
    cmds.reserve(e.commands.size() + 16);
    for (size_t i = 0; i < e.commands.size(); ++i) {
        const EngineCommand& c = e.commands[i];
        if (c.kind != kCmdConcatConv1x1) {
            cmds.push_back(c);
            src.push_back((uint32_t)i);
            continue;
        }
        const std::vector<uint32_t>& p = c.params;
        if (c.inputs.size() < 3 || p.size() < 5 + (c.inputs.size() - 2)) {
            err = "command " + std::to_string(i) + ": malformed CONCAT_CONV1X1";
            return false;
        }
        const size_t k = c.inputs.size() - 2;
        const uint32_t N = p[0], H = p[1], W = p[2], OC = p[3];
        uint64_t sum = 0;
        for (size_t j = 0; j < k; ++j) sum += p[5 + j];
        if (N == 0 || H == 0 || W == 0 || OC == 0 || sum == 0 || sum > 0xFFFFFFu || k > 8) {
            err = "command " + std::to_string(i) + ": bad CONCAT_CONV1X1 geometry";
            return false;
        }
        // the concatenated input as a value of its own
        const uint32_t vid = (uint32_t)e.values.size();
        EngineValue v;
        v.id = vid;
        v.flags = 0;
        v.elements = uint64_t(N) * sum * H * W;
        v.shape4[0] = N, v.shape4[1] = (uint32_t)sum, v.shape4[2] = H, v.shape4[3] = W;
        e.values.push_back(v);
        e.constants.push_back(EngineConstant{});
        e.packed.push_back(EnginePacked{});
        EngineCommand cat;
        cat.kind = kCmdConcat;
        cat.output = vid;
        cat.precision = c.precision;
        cat.inputs.assign(c.inputs.begin(), c.inputs.begin() + k);
        // engine.py CONCAT params: elements, rank, axis, count, shape4, sizes
        cat.params = {(uint32_t)std::min<uint64_t>(v.elements, 0xFFFFFFFFu), 4u, 1u, (uint32_t)k, N, (uint32_t)sum, H, W};
        for (size_t j = 0; j < 8; ++j) cat.params.push_back(p[5 + std::min(j, k - 1)]);
        cat.params.push_back(0u);
        cat.params.push_back(0u);
        cat.plan_flags = kPlanFlagAuthoritative;
        EngineCommand conv;
        conv.kind = p[4] ? kCmdConvSilu : kCmdConv;
        conv.output = c.output;
        conv.precision = c.precision;
        conv.inputs = {vid, c.inputs[k], c.inputs[k + 1]};
        conv.params = {N, (uint32_t)sum, H, W, OC, H, W, 1u, 1u, 1u, 1u, 0u, 0u, 1u, 1u, 1u};
        // plan kernel 3 = the native fp16 concat + 1x1 kernel on the layout-4
        // weight (engine.py:1080-1089): the fp16 1x1 kernel id 45 reads that
        // layout; 1 / 0 (generic fp32 paths) run on the generic kernel
        const uint32_t kern = c.plan_kernel == 3 ? 45u : 5u;
        conv.planned_kernel = kern;
        conv.plan_kernel = kern;
        conv.plan_precision = c.plan_precision;
        conv.packed_value = c.packed_value;
        conv.plan_flags = c.plan_flags;
        cmds.push_back(std::move(cat));
        src.push_back((uint32_t)i);
        cmds.push_back(std::move(conv));
        src.push_back((uint32_t)i);
    }
    e.commands = std::move(cmds);
    e.src_cmd = std::move(src);
    return true;
}

bool parse_engine(const uint8_t* data, size_t size, Engine& out, std::string& err) {
    if (!data || size < 64) {
        err = "truncated AEXRT engine header";
        return false;
    }
    if (std::memcmp(data, kMagic, 8) != 0) {
        err = "not an AEXRT engine (bad magic)";
        return false;
    }
    uint32_t version = 0, header_size = 0, count = 0, flags = 0;
    uint64_t file_size = 0, toc_offset = 0, toc_size = 0;
    rd(data, size, 8, version);
    rd(data, size, 12, header_size);
    rd(data, size, 16, count);
    rd(data, size, 20, flags);
    rd(data, size, 24, file_size);
    rd(data, size, 32, toc_offset);
    rd(data, size, 40, toc_size);
    if (version != 1 || header_size != 64) {
        err = "unsupported AEXRT engine version";
        return false;
    }
    if (file_size != size || toc_size != uint64_t(count) * 32u || toc_offset > size || size - toc_offset < toc_size) {
        err = "AEXRT engine size/TOC mismatch";
        return false;
    }
    Section sec[13];
    for (uint32_t i = 0; i < count; ++i) {
        const size_t e = toc_offset + size_t(i) * 32u;
        uint32_t type = 0, crc = 0;
        uint64_t off = 0, sz = 0;
        rd(data, size, e, type);
        rd(data, size, e + 8, off);
        rd(data, size, e + 16, sz);
        rd(data, size, e + 24, crc);
        if (off > size || size - off < sz) {
            err = "AEXRT section out of range";
            return false;
        }
        if (crc32_ieee(data + off, sz) != crc) {
            err = "AEXRT section " + std::to_string(type) + " checksum mismatch";
            return false;
        }
        if (type >= 1 && type <= 12) sec[type] = Section{data + off, size_t(sz)};
    }
    for (int t = 1; t <= 6; ++t)
        if (!sec[t].data) {
            err = "AEXRT engine lacks section " + std::to_string(t);
            return false;
        }

    // 1: manifest (engine.py:2556-2580)
    {
        const Section& s = sec[1];
        if (s.size < 124) {
            err = "truncated AEXRT manifest";
            return false;
        }
        uint32_t v[17];
        std::memcpy(v, s.data, sizeof(v));
        EngineManifest& m = out.manifest;
        m.precision = v[2];
        m.layout = v[4];
        m.has_objectness = v[5];
        m.channels = v[6];
        m.anchors = v[7];
        m.classes = v[8];
        m.max_candidates = v[9];
        m.max_detections = v[10];
        m.graph_node_count = v[11];
        m.value_count = v[12];
        m.constant_count = v[13];
        m.command_count = v[14];
        m.input_value = v[15];
        m.output_value = v[16];
        std::memcpy(&m.input_elements, s.data + 68, 8);
        std::memcpy(&m.conf_threshold, s.data + 84, 4);
        std::memcpy(&m.iou_threshold, s.data + 88, 4);
    }
    // 2: values (engine.py:2583-2598)
    {
        const Section& s = sec[2];
        uint32_t n = 0;
        if (!rd(s.data, s.size, 0, n) || s.size < 8 + size_t(n) * 48u) {
            err = "truncated AEXRT values section";
            return false;
        }
        out.values.resize(n);
        for (uint32_t i = 0; i < n; ++i) {
            const uint8_t* r = s.data + 8 + size_t(i) * 48u;
            EngineValue v;
            std::memcpy(&v.id, r, 4);
            std::memcpy(&v.flags, r + 4, 4);
            std::memcpy(&v.elements, r + 8, 8);
            std::memcpy(v.shape4, r + 16, 16);
            if (v.id >= n) {
                err = "AEXRT value id out of range";
                return false;
            }
            out.values[v.id] = v;
        }
    }
    const uint32_t nvals = uint32_t(out.values.size());
    // 3: commands (engine.py:2601-2617)
    {
        const Section& s = sec[3];
        uint32_t n = 0;
        if (!rd(s.data, s.size, 0, n)) {
            err = "truncated AEXRT commands section";
            return false;
        }
        size_t off = 8;
        out.commands.resize(n);
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t h[6];
            if (off > s.size || s.size - off < sizeof(h)) {
                err = "truncated AEXRT command record";
                return false;
            }
            std::memcpy(h, s.data + off, sizeof(h));
            off += sizeof(h);
            EngineCommand& c = out.commands[i];
            c.kind = h[0];
            c.output = h[1];
            c.planned_kernel = h[4];
            c.precision = h[5];
            const size_t need = (size_t(h[2]) + h[3]) * 4u;
            if (h[2] > 64 || h[3] > 256 || s.size - off < need) {
                err = "truncated AEXRT command operands";
                return false;
            }
            c.inputs.resize(h[2]);
            c.params.resize(h[3]);
            if (h[2]) std::memcpy(c.inputs.data(), s.data + off, h[2] * 4u);
            off += h[2] * 4u;
            if (h[3]) std::memcpy(c.params.data(), s.data + off, h[3] * 4u);
            off += h[3] * 4u;
            if (c.output >= nvals) {
                err = "AEXRT command output out of range";
                return false;
            }
            for (uint32_t v : c.inputs)
                if (v >= nvals) {
                    err = "AEXRT command input out of range";
                    return false;
                }
        }
    }
    // 4: constants (engine.py:2620-2647)
    out.constants.assign(nvals, EngineConstant{});
    {
        const Section& s = sec[4];
        uint32_t n = 0;
        if (!rd(s.data, s.size, 0, n) || s.size < 8 + size_t(n) * 32u) {
            err = "truncated AEXRT constants section";
            return false;
        }
        for (uint32_t i = 0; i < n; ++i) {
            const uint8_t* r = s.data + 8 + size_t(i) * 32u;
            uint32_t id, prec;
            uint64_t elements, off, nbytes;
            std::memcpy(&id, r, 4);
            std::memcpy(&prec, r + 4, 4);
            std::memcpy(&elements, r + 8, 8);
            std::memcpy(&off, r + 16, 8);
            std::memcpy(&nbytes, r + 24, 8);
            const uint64_t esz = prec == 2 ? 2 : 4;
            if (id >= nvals || off > s.size || s.size - off < nbytes || nbytes != elements * esz) {
                err = "invalid AEXRT constant record";
                return false;
            }
            EngineConstant& c = out.constants[id];
            c.precision = prec;
            c.elements = elements;
            c.raw.assign(s.data + off, s.data + off + nbytes);
            c.present = true;
        }
    }
    // 5: kernel plan (engine.py:2650-2662)
    {
        const Section& s = sec[5];
        uint32_t n = 0;
        if (!rd(s.data, s.size, 0, n) || s.size < 8 + size_t(n) * 24u || n != out.commands.size()) {
            err = "AEXRT kernel plan does not cover the command stream";
            return false;
        }
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t r[6];
            std::memcpy(r, s.data + 8 + size_t(i) * 24u, sizeof(r));
            if (r[0] != i || r[1] != out.commands[i].kind) {
                err = "AEXRT kernel plan record does not match its command";
                return false;
            }
            EngineCommand& c = out.commands[i];
            c.plan_kernel = r[2];
            c.plan_precision = r[3];
            c.packed_value = r[4];
            c.plan_flags = r[5];
            if (c.packed_value != UINT32_MAX && c.packed_value >= nvals) {
                err = "AEXRT kernel plan packed value out of range";
                return false;
            }
        }
    }
    // 6: packed weights (engine.py:2665-2690)
    out.packed.assign(nvals, EnginePacked{});
    {
        const Section& s = sec[6];
        uint32_t n = 0;
        if (!rd(s.data, s.size, 0, n) || s.size < 8 + size_t(n) * 40u) {
            err = "truncated AEXRT packed weights section";
            return false;
        }
        for (uint32_t i = 0; i < n; ++i) {
            const uint8_t* r = s.data + 8 + size_t(i) * 40u;
            uint32_t h[4];
            uint64_t elements, off, nbytes;
            std::memcpy(h, r, 16);
            std::memcpy(&elements, r + 16, 8);
            std::memcpy(&off, r + 24, 8);
            std::memcpy(&nbytes, r + 32, 8);
            if (h[0] >= nvals || off > s.size || s.size - off < nbytes) {
                err = "invalid AEXRT packed weight record";
                return false;
            }
            EnginePacked& p = out.packed[h[0]];
            p.layout = h[1];
            p.in_channels = h[2];
            p.out_channels = h[3];
            p.elements = elements;
            p.data.assign(s.data + off, s.data + off + nbytes);
            p.present = true;
        }
    }
    // fail-closed plan <-> packed-weight coherence for the int8 kernels
    // (native/aexrt_d3d12_runtime.cpp:18132-18164)
    for (size_t i = 0; i < out.commands.size(); ++i) {
        const EngineCommand& c = out.commands[i];
        const bool int8 = c.plan_kernel == 51 || c.plan_kernel == 52 || c.plan_kernel == 53;
        if (!int8 || c.packed_value == UINT32_MAX) continue;
        const EnginePacked& p = out.packed[c.packed_value];
        const uint32_t kk = c.plan_kernel == 51 ? 1u : 9u;
        if (c.params.size() < 16 || !p.present || p.layout != 8 || p.in_channels != c.params[1] ||
            p.out_channels != c.params[4] || p.elements != uint64_t(c.params[1]) * c.params[4] * kk ||
            p.data.size() != p.elements + 4ull * c.params[4]) {
            err = "command " + std::to_string(i) + ": planned int8 kernel without a matching layout-8 weight";
            return false;
        }
    }
    if (out.manifest.input_value >= nvals || out.manifest.output_value >= nvals) {
        err = "AEXRT manifest input/output value out of range";
        return false;
    }
    return true;
}

}  // namespace aexrt
