// .aexrt container parser.  Every offset and size is checked against the
// buffer before it is read, every section's CRC32 is verified, and an engine
// the reference loader would refuse is refused here too (fail closed).
#include <algorithm>
#include <cstring>
#include <string>

#include "runtime.h"

namespace aexrt {

namespace {

constexpr char kMagic[8] = {'A', 'E', 'X', 'R', 'T', 'E', 'N', 'G'};

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

namespace {

// Bounds-checked little-endian cursor over one section.
struct Cursor {
    const uint8_t* p;
    size_t n, at = 0;
    Cursor(const uint8_t* data, size_t size) : p(data), n(size) {}
    template <typename T>
    bool get(T& v) {
        if (at > n || n - at < sizeof(T)) return false;
        std::memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return true;
    }
    template <typename... T>
    bool all(T&... v) { return (get(v) && ...); }
    bool skip(size_t k) {
        if (at > n || n - at < k) return false;
        at += k;
        return true;
    }
    bool done() const { return at == n; }
};

bool valid_kind(uint32_t k) { return k >= kCmdConv && k <= kCmdSoftmax; }

// Kernel ids of the runtime enum (RT:8881-8940) used by the plan checks.
bool conv_reads_packed_weight(uint32_t kernel, uint32_t precision, uint32_t flags) {
    switch (kernel) {
        case 32: case 33: case 34: case 39: case 43: case 44: case 45: case 47: case 48: case 49: case 50:
        case 51: case 52: case 53:
            return true;
        case 40: case 46:
            return precision == 2 && (flags & 2u);
        case 54:
            return (flags & 2u) != 0;
        default:
            return false;
    }
}

bool fail(std::string& err, const std::string& what) {
    err = what;
    return false;
}

}  // namespace

// The acceptance rules of the reference loader, parse_aexrt_engine
// (native/aexrt_d3d12_runtime.cpp:17560-18590), restated: header and TOC
// (17560-17599), manifest (17605-17621), values (17645-17689), commands
// (17691-17733), constants (17735-17764), kernel plan (17766-17887), memory
// plan V2/V1 (17889-17982), packed weights (17984-18264), fusion plan
// (18266-18325), pipeline cache (18556-18590), output channels (18592-18593).
// Sections 10 and 11 are accepted when present with their prerequisites;
// their contents (the D3D12 dispatch and barrier schedule) are not used.
bool parse_engine(const uint8_t* data, size_t size, Engine& out, std::string& err) {
    if (!data || size < 64) return fail(err, "truncated AEXRT engine header");
    if (std::memcmp(data, kMagic, 8) != 0) return fail(err, "not an AEXRT engine (bad magic)");
    Cursor h(data + 8, size - 8);
    uint32_t version = 0, header_size = 0, count = 0, flags = 0;
    uint64_t file_size = 0, toc_offset = 0, toc_size = 0;
    h.all(version, header_size, count, flags, file_size, toc_offset, toc_size);
    if (version != 1 || header_size != 64) return fail(err, "unsupported AEXRT engine version");
    if (count == 0 || count > 64 || file_size != size || toc_size != uint64_t(count) * 32u || toc_offset > size ||
        size - toc_offset < toc_size)
        return fail(err, "AEXRT engine size/TOC mismatch");
    if ((flags & 1u) == 0) return fail(err, "AEXRT engine header flag bit 0 clear");
    Section sec[13];
    Cursor toc(data + toc_offset, size_t(toc_size));
    for (uint32_t i = 0; i < count; ++i) {
        uint32_t type = 0, sflags = 0, crc = 0, reserved = 0;
        uint64_t off = 0, sz = 0;
        toc.all(type, sflags, off, sz, crc, reserved);
        if (reserved != 0) return fail(err, "AEXRT TOC entry with a nonzero reserved field");
        if (off > size || size - off < sz) return fail(err, "AEXRT section out of range");
        if (crc32_ieee(data + off, sz) != crc)
            return fail(err, "AEXRT section " + std::to_string(type) + " checksum mismatch");
        if (type >= 1 && type <= 12) {
            if (sec[type].data) return fail(err, "duplicate AEXRT section " + std::to_string(type));
            sec[type] = Section{data + off, size_t(sz)};
        }
    }
    for (int t = 1; t <= 9; ++t)
        if (!sec[t].data) return fail(err, "AEXRT engine lacks section " + std::to_string(t));
    uint32_t mem_version = 0;
    if (sec[7].size < 4) return fail(err, "truncated AEXRT memory plan");
    std::memcpy(&mem_version, sec[7].data, 4);
    const bool mem_v2 = mem_version == 2u;

    // 1: manifest
    EngineManifest& m = out.manifest;
    {
        Cursor c(sec[1].data, sec[1].size);
        uint32_t v[17];
        for (uint32_t& x : v)
            if (!c.get(x)) return fail(err, "truncated AEXRT manifest");
        if (!c.all(m.input_elements, m.arena_nbytes, m.conf_threshold, m.iou_threshold) || !c.skip(32))
            return fail(err, "truncated AEXRT manifest");
        if (v[0] != 1 || v[1] != 1 || (v[2] != 1 && v[2] != 2) || v[3] != 2 || (v[4] != 1 && v[4] != 2) || v[5] > 1 ||
            v[6] == 0 || v[7] == 0 || v[8] == 0 || v[12] == 0 || v[14] == 0 || v[15] >= v[12] || v[16] >= v[12] ||
            m.input_elements == 0 || m.arena_nbytes == 0)
            return fail(err, "invalid AEXRT manifest");
        m.precision = v[2], m.layout = v[4], m.has_objectness = v[5], m.channels = v[6], m.anchors = v[7];
        m.classes = v[8], m.max_candidates = v[9], m.max_detections = v[10], m.graph_node_count = v[11];
        m.value_count = v[12], m.constant_count = v[13], m.command_count = v[14], m.input_value = v[15];
        m.output_value = v[16];
    }
    // 2: values
    std::vector<uint64_t> arena_off, arena_bytes;
    {
        Cursor c(sec[2].data, sec[2].size);
        uint32_t n = 0, reserved = 0;
        if (!c.all(n, reserved) || reserved != 0 || n != m.value_count) return fail(err, "invalid AEXRT values header");
        out.values.resize(n);
        arena_off.assign(n, UINT64_MAX);
        arena_bytes.assign(n, 0);
        for (uint32_t i = 0; i < n; ++i) {
            EngineValue& v = out.values[i];
            uint64_t off = 0, nb = 0;
            if (!c.all(v.id, v.flags, v.elements, v.shape4[0], v.shape4[1], v.shape4[2], v.shape4[3], off, nb))
                return fail(err, "truncated AEXRT values section");
            if (v.id != i || v.elements == 0) return fail(err, "AEXRT value record out of order or empty");
            const bool arena = (v.flags & 4u) != 0, alias = (v.flags & 8u) != 0, konst = (v.flags & 2u) != 0;
            if (arena) {
                const bool sized = mem_v2 ? (nb == v.elements * 4u || nb == v.elements * 2u) : nb == v.elements * 4u;
                if (off == UINT64_MAX || !sized || off > m.arena_nbytes || nb > m.arena_nbytes - off)
                    return fail(err, "AEXRT arena value outside the arena");
            } else if (!mem_v2 && !alias && !konst) {
                return fail(err, "AEXRT value without storage under a V1 memory plan");
            } else if (off != UINT64_MAX || nb != 0) {
                return fail(err, "AEXRT non-arena value with an arena range");
            }
            arena_off[i] = off, arena_bytes[i] = nb;
        }
        if (!c.done()) return fail(err, "trailing bytes in the AEXRT values section");
    }
    const uint32_t nvals = uint32_t(out.values.size());
    // 3: commands
    {
        Cursor c(sec[3].data, sec[3].size);
        uint32_t n = 0, reserved = 0;
        if (!c.all(n, reserved) || reserved != 0 || n != m.command_count)
            return fail(err, "invalid AEXRT commands header");
        out.commands.resize(n);
        for (uint32_t i = 0; i < n; ++i) {
            EngineCommand& cmd = out.commands[i];
            uint32_t ni = 0, np = 0;
            if (!c.all(cmd.kind, cmd.output, ni, np, cmd.planned_kernel, cmd.precision))
                return fail(err, "truncated AEXRT command record");
            const uint32_t k = cmd.kind, pk = cmd.planned_kernel;
            if (!valid_kind(k) || cmd.output >= nvals || ni > 32 || np > 128 || (cmd.precision != 1 && cmd.precision != 2))
                return fail(err, "invalid AEXRT command " + std::to_string(i));
            if ((k == kCmdConv || k == kCmdConvSilu) && (pk > 54 || (pk >= 48 && pk <= 50)))
                return fail(err, "AEXRT command " + std::to_string(i) + ": conv kernel id not accepted");
            if ((k == kCmdConcatConv1x1 && pk > 3) || (k > kCmdConcatConv1x1 && pk != 0))
                return fail(err, "AEXRT command " + std::to_string(i) + ": kernel id for a non-conv command");
            cmd.inputs.resize(ni);
            cmd.params.resize(np);
            for (uint32_t& v : cmd.inputs)
                if (!c.get(v) || v >= nvals) return fail(err, "AEXRT command input out of range");
            for (uint32_t& v : cmd.params)
                if (!c.get(v)) return fail(err, "truncated AEXRT command operands");
        }
        if (!c.done()) return fail(err, "trailing bytes in the AEXRT commands section");
    }
    // 4: constants
    out.constants.assign(nvals, EngineConstant{});
    {
        const Section& s = sec[4];
        Cursor c(s.data, s.size);
        uint32_t n = 0, reserved = 0;
        if (!c.all(n, reserved) || reserved != 0 || n != m.constant_count)
            return fail(err, "invalid AEXRT constants header");
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t id = 0, prec = 0;
            uint64_t elements = 0, off = 0, nb = 0;
            if (!c.all(id, prec, elements, off, nb)) return fail(err, "truncated AEXRT constants section");
            if (id >= nvals || (prec != 1 && prec != 2) || elements != out.values[id].elements ||
                nb != elements * (prec == 2 ? 2u : 4u) || off > s.size || nb > s.size - off ||
                (out.values[id].flags & 2u) == 0)
                return fail(err, "invalid AEXRT constant record");
            EngineConstant& k = out.constants[id];
            k.precision = prec;
            k.elements = elements;
            k.raw.assign(s.data + off, s.data + off + nb);
            k.present = true;
        }
    }
    // 5: kernel plan
    {
        Cursor c(sec[5].data, sec[5].size);
        uint32_t n = 0, plan_version = 0;
        if (!c.all(n, plan_version) || n != out.commands.size() || plan_version != 1)
            return fail(err, "AEXRT kernel plan does not cover the command stream");
        for (uint32_t i = 0; i < n; ++i) {
            EngineCommand& cmd = out.commands[i];
            uint32_t idx = 0, kind = 0;
            if (!c.all(idx, kind, cmd.plan_kernel, cmd.plan_precision, cmd.packed_value, cmd.plan_flags))
                return fail(err, "truncated AEXRT kernel plan");
            const uint32_t pf = cmd.plan_flags, pk = cmd.plan_kernel;
            if (idx != i || kind != cmd.kind || (cmd.plan_precision != 1 && cmd.plan_precision != 2) || !(pf & 1u) ||
                (pf & ~31u) || pk != cmd.planned_kernel || cmd.plan_precision != cmd.precision)
                return fail(err, "AEXRT kernel plan record does not match its command");
            const bool conv = kind == kCmdConv || kind == kCmdConvSilu;
            const bool concat_packed = kind == kCmdConcatConv1x1 && pk == 3;
            const bool wants = (conv && conv_reads_packed_weight(pk, cmd.plan_precision, pf)) || concat_packed;
            if (wants) {
                const size_t ni = cmd.inputs.size();
                const uint32_t expect = ni >= 2 ? (concat_packed ? cmd.inputs[ni - 2] : cmd.inputs[1]) : UINT32_MAX;
                if (cmd.packed_value != expect)
                    return fail(err, "command " + std::to_string(i) + ": kernel plan names the wrong packed weight");
            } else if (cmd.packed_value != UINT32_MAX) {
                return fail(err, "command " + std::to_string(i) + ": packed weight on a kernel that reads none");
            }
            const bool native_fp16 = (kind == kCmdConvSilu && (pk == 43 || pk == 44 || pk == 47 || pk == 48 ||
                                                               ((pk == 40 || pk == 46) && (pf & 2u)))) ||
                                     (conv && pk == 45) || concat_packed;
            if (native_fp16 && (cmd.plan_precision != 2 || !(pf & 2u)))
                return fail(err, "command " + std::to_string(i) + ": native fp16 kernel without fp16 DXIL plan");
        }
    }
    // 7: memory plan
    {
        Cursor c(sec[7].data, sec[7].size);
        if (mem_v2) {
            uint32_t ver = 0, align = 0, pages = 0, nrec = 0, pflags = 0, reserved = 0;
            uint64_t total = 0;
            if (!c.all(ver, align, pages, nrec, total, pflags, reserved) || align < 4 || (align & (align - 1)) ||
                pages == 0 || pages > 64 || nrec > nvals || total != m.arena_nbytes || pflags != 1 || reserved != 0)
                return fail(err, "invalid AEXRT memory plan header");
            std::vector<uint32_t> pdtype(pages), playout(pages);
            std::vector<uint64_t> psize(pages);
            uint64_t sum = 0;
            for (uint32_t p = 0; p < pages; ++p) {
                uint32_t id = 0, dt = 0, lay = 0, fl = 0;
                uint64_t nb = 0;
                if (!c.all(id, dt, lay, fl, nb) || id != p || (dt != 1 && dt != 2) || (lay != 1 && lay != 2) ||
                    (lay == 2 && dt != 2) || fl != 1 || nb == 0 || nb % align || nb > total - sum)
                    return fail(err, "invalid AEXRT memory page");
                pdtype[p] = dt, playout[p] = lay, psize[p] = nb;
                sum += nb;
            }
            if (sum != total) return fail(err, "AEXRT memory pages do not add up to the arena");
            uint32_t expect = 0;
            for (uint32_t i = 0; i < nvals; ++i) expect += arena_off[i] != UINT64_MAX && !(out.values[i].flags & 2u);
            if (nrec != expect) return fail(err, "AEXRT memory plan does not cover the arena values");
            std::vector<uint8_t> seen(nvals, 0);
            for (uint32_t r = 0; r < nrec; ++r) {
                uint32_t vid = 0, vf = 0, page = 0, dt = 0, lay = 0, res = 0;
                uint64_t off = 0, nb = 0;
                if (!c.all(vid, vf, page, dt, lay, res, off, nb) || vid >= nvals || seen[vid] || !(vf & 4u) ||
                    page >= pages || res != 0)
                    return fail(err, "invalid AEXRT memory value record");
                if (dt != pdtype[page] || lay != playout[page] || arena_off[vid] != off || arena_bytes[vid] != nb ||
                    nb != out.values[vid].elements * (dt == 2 ? 2u : 4u) || off % align || off > psize[page] ||
                    nb > psize[page] - off)
                    return fail(err, "AEXRT memory value record disagrees with its page or value");
                seen[vid] = 1;
            }
            if (!c.done()) return fail(err, "trailing bytes in the AEXRT memory plan");
            out.extras.memory_plan_version = 2;
            out.extras.arena_pages = pages;
        } else {
            uint32_t align = 0, n = 0;
            uint64_t total = 0;
            if (!c.all(align, n, total) || align < 4 || (align & (align - 1)) || total != m.arena_nbytes)
                return fail(err, "invalid AEXRT V1 memory plan");
            for (uint32_t r = 0; r < n; ++r) {
                uint32_t vid = 0, vf = 0;
                uint64_t off = 0, nb = 0;
                if (!c.all(vid, vf, off, nb) || vid >= nvals || !(vf & 4u) || arena_off[vid] != off ||
                    arena_bytes[vid] != nb)
                    return fail(err, "invalid AEXRT V1 memory record");
            }
            if (!c.done()) return fail(err, "trailing bytes in the AEXRT memory plan");
            out.extras.memory_plan_version = 1;
            out.extras.arena_pages = 1;
        }
    }
    // 6: packed weights
    out.packed.assign(nvals, EnginePacked{});
    {
        const Section& s = sec[6];
        Cursor c(s.data, s.size);
        uint32_t n = 0, reserved = 0;
        if (!c.all(n, reserved) || reserved != 0) return fail(err, "invalid AEXRT packed weights header");
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t vid = 0, layout = 0, ic = 0, oc = 0;
            uint64_t elements = 0, off = 0, nb = 0;
            if (!c.all(vid, layout, ic, oc, elements, off, nb)) return fail(err, "truncated AEXRT packed weights");
            if (vid >= nvals || layout < 1 || layout > 9 || ic == 0 || oc == 0)
                return fail(err, "invalid AEXRT packed weight record");
            const uint64_t icoc = uint64_t(ic) * oc;
            const uint64_t kk = (layout == 3 || layout == 5) ? 16u
                                : layout == 4                 ? 1u
                                : layout == 8                 ? elements / icoc
                                : layout == 9                 ? 36u
                                                              : 9u;
            const uint64_t esz = (layout == 1 || layout == 5 || layout == 7) ? 4u : layout == 8 ? 1u : 2u;
            const bool shape_ok =
                !(layout == 4 && (ic % 4 || oc % 8)) && !((layout == 6 || layout == 7) && (ic % 4 || oc % 4)) &&
                !(layout == 8 && (ic % 4 || oc % 4 || elements % 4 || (kk != 1 && kk != 9) ||
                                  nb != elements + uint64_t(oc) * 4u)) &&
                elements == icoc * kk && (layout == 8 || nb == elements * esz);
            if (!shape_ok || off > s.size || nb > s.size - off)
                return fail(err, "invalid AEXRT packed weight record");
            EnginePacked& p = out.packed[vid];
            if (p.present) return fail(err, "two AEXRT packed weights for one value");
            if (!(out.values[vid].flags & 2u)) return fail(err, "AEXRT packed weight for a non-constant value");
            p.layout = layout, p.in_channels = ic, p.out_channels = oc, p.elements = elements;
            p.data.assign(s.data + off, s.data + off + nb);
            p.present = true;
        }
    }
    // every kernel-plan packed weight has the layout its kernel reads
    for (size_t i = 0; i < out.commands.size(); ++i) {
        const EngineCommand& c = out.commands[i];
        if (c.packed_value == UINT32_MAX) continue;
        const EnginePacked& p = out.packed[c.packed_value];
        const std::string where = "command " + std::to_string(i) + ": ";
        const uint32_t pk = c.plan_kernel;
        if (c.kind == kCmdConcatConv1x1) {
            const size_t k = c.inputs.size() >= 2 ? c.inputs.size() - 2 : 0;
            if (k == 0 || c.params.size() < 5 + k) return fail(err, where + "malformed CONCAT_CONV1X1");
            uint64_t sum = 0;
            for (size_t j = 0; j < k; ++j) sum += c.params[5 + j];
            if (!p.present || p.layout != 4 || p.in_channels != sum || p.out_channels != c.params[3])
                return fail(err, where + "concat 1x1 plan without a matching layout-4 weight");
            continue;
        }
        if (c.params.size() < 16) return fail(err, where + "conv with fewer than 16 params");
        const uint32_t ic = c.params[1], oc = c.params[4];
        uint32_t want = 0;
        if (pk == 51 || pk == 52 || pk == 53) {
            const uint32_t kk = pk == 51 ? 1u : 9u;
            if (!p.present || p.layout != 8 || p.in_channels != ic || p.out_channels != oc ||
                p.elements != uint64_t(ic) * oc * kk || p.data.size() != p.elements + 4ull * oc)
                return fail(err, where + "planned int8 kernel without a matching layout-8 weight");
            continue;
        }
        if (pk == 54) want = 9;
        else if (pk == 46) want = 5;
        else if (pk == 40) want = 3;
        else if (pk == 45) want = 4;
        else if (pk == 47 || pk == 48) want = 6;
        else if (pk == 50) want = 7;
        const bool direct_pack4 = want == 0 && p.present && (p.layout == 1 || p.layout == 2);
        if (!p.present || (want && p.layout != want) || (!want && !direct_pack4) || p.in_channels != ic ||
            p.out_channels != oc)
            return fail(err, where + "kernel plan weight has the wrong packed layout or shape");
        if ((pk == 43 || pk == 44) && p.layout != 2) return fail(err, where + "native fp16 kernel without fp16 weight");
        if (pk == 46) {
            static const uint32_t shape46[16] = {1, 256, 10, 10, 256, 10, 10, 3, 3, 1, 1, 1, 1, 1, 1, 1};
            if (!std::equal(shape46, shape46 + 16, c.params.begin()))
                return fail(err, where + "kernel 46 outside its measured 256x256 10x10 shape");
        }
    }
    // 8: fusion plan
    {
        Cursor c(sec[8].data, sec[8].size);
        uint32_t ver = 0, n = 0, ncmd = 0, fflags = 0;
        const uint32_t cmds = uint32_t(out.commands.size());
        if (!c.all(ver, n, ncmd, fflags) || ver != 1 || ncmd != cmds || n > ncmd * 2u || !(fflags & 1u))
            return fail(err, "invalid AEXRT fusion plan header");
        for (uint32_t g = 0; g < n; ++g) {
            uint32_t kind = 0, a = 0, b = 0, prec = 0, kern = 0, gf = 0, aux0 = 0, aux1 = 0;
            if (!c.all(kind, a, b, prec, kern, gf, aux0, aux1) || kind < 1 || kind > 9 || a >= cmds || b >= cmds ||
                a > b || (prec != 1 && prec != 2) || !(gf & 1u))
                return fail(err, "invalid AEXRT fusion group");
            if (kind == 1) {
                static const uint32_t shape[16] = {1, 256, 10, 10, 64, 10, 10, 3, 3, 1, 1, 1, 1, 1, 1, 1};
                const EngineCommand &x = out.commands[a], &y = out.commands[b];
                if (b != a + 1 || prec != 2 || kern != 40 || gf != 3 || aux0 || aux1 || x.kind != kCmdConvSilu ||
                    y.kind != kCmdConvSilu || x.inputs.size() < 3 || y.inputs.size() < 3 ||
                    x.inputs[0] != y.inputs[0] || x.output == y.output || x.params.size() < 16 ||
                    y.params.size() < 16 || !std::equal(shape, shape + 16, x.params.begin()) ||
                    !std::equal(shape, shape + 16, y.params.begin()))
                    return fail(err, "invalid paired-3x3 fusion group");
                for (uint32_t w : {x.inputs[1], y.inputs[1]}) {
                    const EnginePacked& p = out.packed[w];
                    if (!p.present || p.layout != 3 || p.in_channels != 256 || p.out_channels != 64)
                        return fail(err, "paired-3x3 fusion group without its Winograd weights");
                }
            } else if (kind == 9) {
                const uint32_t dim = aux0 & 0xffffu, hidden = aux0 >> 16, entry = aux1 & 0xffffu, outc = aux1 >> 16;
                const bool measured = (dim == 20 && entry == 512 && hidden == 128 && outc == 256) ||
                                      (dim == 40 && entry == 256 && hidden == 64 && outc == 128) ||
                                      (dim == 20 && entry == 256 && hidden == 128 && outc == 256);
                if (b != a + 5 || prec != 2 || kern != 0 || gf != 3 || !measured)
                    return fail(err, "invalid LatticeChain fusion group");
            }
        }
        if (!c.done()) return fail(err, "trailing bytes in the AEXRT fusion plan");
        out.extras.fusion_groups = n;
    }
    // 9: pipeline cache
    {
        const Section& s = sec[9];
        Cursor c(s.data, s.size);
        uint32_t ver = 0, ndxil = 0, npso = 0, cflags = 0;
        if (!c.all(ver, ndxil, npso, cflags) || ver != 1 || uint64_t(ndxil) + npso > 4096u)
            return fail(err, "invalid AEXRT pipeline cache header");
        for (uint32_t r = 0; r < ndxil + npso; ++r) {
            uint32_t kind = 0, rf = 0;
            uint64_t key = 0, off = 0, nb = 0;
            if (!c.all(kind, rf, key, off, nb) || (kind != 1 && kind != 2) || key == 0 || nb == 0 ||
                (kind == 1 && (rf & ~1u)) || (kind == 2 && rf) || off > s.size || nb > s.size - off)
                return fail(err, "invalid AEXRT pipeline cache record");
        }
        out.extras.cache_records = ndxil + npso;
    }
    if (m.classes + (m.has_objectness ? 5u : 4u) > m.channels)
        return fail(err, "AEXRT manifest classes exceed the output channels");
    if (sec[11].data && (!mem_v2 || !sec[10].data))
        return fail(err, "AEXRT barrier plan without a V2 memory plan and a physical dispatch plan");
    out.extras.physical_dispatch_plan = sec[10].data != nullptr;
    out.extras.barrier_plan = sec[11].data != nullptr;
    return true;
}

}  // namespace aexrt
