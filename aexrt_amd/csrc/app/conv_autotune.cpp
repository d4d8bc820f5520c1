// conv_autotune: per-device choice of each conv's kernel algorithm for an
// .aexrt engine, over the library's public C ABI (the counterpart of the
// reference's examples/cpp/conv_autotune.cpp, its --emit-map JSON consumed by
// `aexrtc build --algo-map`, src/aexrt/cli.py:92-93).
//
// For every distinct conv shape the tool overrides the algorithm of one of
// its commands with each candidate the runtime reports, checks that the
// network's detections stay those of the baseline run (same count, scores
// within 1e-3, boxes within 0.05 px), and times that command with the
// runtime's per-step events.  A candidate replaces the planned algorithm
// only when its median time is at least 5% lower.  All winners are then
// applied together; if the combination fails to run or to pass the gate,
// winners are dropped one at a time until it does.  Outputs: a markdown
// report, a JSON map {engine command index: algorithm} and a C header table.
//
// Usage: conv_autotune engine.aexrt [--device N] [--runs N] [--warmup N]
//                      [--limit K] [--out report.md] [--emit-map map.json]
//                      [--emit-header tuned.h]
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "aexrt_hip.h"

namespace {

double wall_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

double median(std::vector<double> v) {
    if (v.empty()) return -1.0;
    std::sort(v.begin(), v.end());
    const size_t h = v.size() / 2;
    return v.size() % 2 ? v[h] : 0.5 * (v[h - 1] + v[h]);
}

// Convs of one shape share a measurement (grouped convs and dilations are
// part of the key: their weights are laid out differently).
using Shape = std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                         uint32_t, uint32_t, uint32_t, uint32_t>;

Shape shape_of(const AexrtConvPlanInfo& p) {
    const AexrtConv2DDesc& d = p.desc;
    return Shape{p.kind_is_silu, d.batch, d.in_channels, d.in_h, d.in_w, d.out_channels, d.out_h, d.out_w,
                 d.kernel_h, d.stride_h, d.pad_top, d.groups, d.dilation_h};
}

std::string shape_str(const AexrtConvPlanInfo& p) {
    const AexrtConv2DDesc& d = p.desc;
    std::ostringstream s;
    s << (p.kind_is_silu ? "silu " : "lin ") << d.batch << "x" << d.in_channels << "x" << d.in_h << "x" << d.in_w
      << " -> " << d.out_channels << "x" << d.out_h << "x" << d.out_w << " k" << d.kernel_h << " s" << d.stride_h
      << " g" << d.groups;
    return s.str();
}

struct Candidate {
    uint32_t algorithm = 0;
    bool ran = false, gate = false;
    double ms = -1.0;
};

struct Row {
    AexrtConvPlanInfo info{};
    double current_ms = -1.0, best_ms = -1.0;
    uint32_t best = 0;
    std::vector<Candidate> cands;
};

struct Tuner {
    AexrtDevice* dev = nullptr;
    AexrtYoloModel* model = nullptr;
    std::vector<float> input;
    uint32_t warmup = 2, runs = 10;
    bool failed = false;

    // one run: wall time, detections into dets
    double run(std::vector<AexrtYoloDetection>& dets) {
        dets.resize(256);
        uint32_t n = 0;
        const double t0 = wall_ms();
        const int ok = aexrt_yolo_run(dev, model, input.data(), input.size(), dets.data(), 256, &n);
        const double t1 = wall_ms();
        failed = ok == 0;
        dets.resize(failed ? 0 : n);
        return failed ? -1.0 : t1 - t0;
    }

    // this command's step time of the last run ("cmd#<index> " label prefix)
    double step_ms(uint32_t command_index) const {
        const std::string prefix = "cmd#" + std::to_string(command_index) + " ";
        const uint32_t n = aexrt_yolo_profile_event_count(model);
        for (uint32_t i = 0; i < n; ++i) {
            const char* label = aexrt_yolo_profile_event_label(model, i);
            if (label && std::strncmp(label, prefix.c_str(), prefix.size()) == 0)
                return aexrt_yolo_profile_event_ms(model, i);
        }
        return -1.0;
    }

    double timed_step(uint32_t command_index) {
        std::vector<AexrtYoloDetection> d;
        std::vector<double> t;
        for (uint32_t i = 0; i < warmup + runs; ++i) {
            if (run(d) < 0) return -1.0;
            const double ms = step_ms(command_index);
            if (i >= warmup && ms >= 0) t.push_back(ms);
        }
        return median(t);
    }
};

bool same_detections(const std::vector<AexrtYoloDetection>& a, const std::vector<AexrtYoloDetection>& b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i) {
        if (std::fabs(a[i].score - b[i].score) > 1e-3f || a[i].class_id != b[i].class_id) return false;
        if (std::fabs(a[i].x1 - b[i].x1) > 0.05f || std::fabs(a[i].y1 - b[i].y1) > 0.05f ||
            std::fabs(a[i].x2 - b[i].x2) > 0.05f || std::fabs(a[i].y2 - b[i].y2) > 0.05f)
            return false;
    }
    return true;
}

int usage() {
    std::fprintf(stderr,
                 "usage: conv_autotune engine.aexrt [--device N] [--runs N] [--warmup N] [--limit K]\n"
                 "                     [--out report.md] [--emit-map map.json] [--emit-header tuned.h]\n");
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    std::string engine, out_path = "conv_autotune_report.md", map_path, header_path;
    uint32_t device_index = 0, limit = 0;
    Tuner t;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&]() -> const char* { return i + 1 < argc ? argv[++i] : nullptr; };
        const char* v = nullptr;
        if (a == "--device" && (v = value())) device_index = (uint32_t)std::strtoul(v, nullptr, 0);
        else if (a == "--runs" && (v = value())) t.runs = std::max(1ul, std::strtoul(v, nullptr, 0));
        else if (a == "--warmup" && (v = value())) t.warmup = (uint32_t)std::strtoul(v, nullptr, 0);
        else if (a == "--limit" && (v = value())) limit = (uint32_t)std::strtoul(v, nullptr, 0);
        else if (a == "--out" && (v = value())) out_path = v;
        else if (a == "--emit-map" && (v = value())) map_path = v;
        else if (a == "--emit-header" && (v = value())) header_path = v;
        else if (!a.empty() && a[0] != '-' && engine.empty()) engine = a;
        else return usage();
    }
    if (engine.empty()) return usage();

    t.dev = aexrt_hip_create_device(device_index);
    if (!t.dev) {
        std::fprintf(stderr, "device %u: %s\n", device_index, aexrt_hip_get_last_error());
        return 2;
    }
    t.model = aexrt_yolo_load_engine(t.dev, engine.c_str());
    if (!t.model || !aexrt_yolo_is_executable(t.model)) {
        std::fprintf(stderr, "load %s: %s\n", engine.c_str(), aexrt_hip_get_last_error());
        aexrt_hip_destroy_device(t.dev);
        return 2;
    }
    // per-step events for the timings; every run then launches its steps one
    // by one on the model stream
    aexrt_yolo_set_profiling(t.model, 1);

    // deterministic input in [-1, 1) (xorshift32)
    t.input.resize(aexrt_yolo_input_element_count(t.model));
    uint32_t st = 0x2545F491u;
    for (float& x : t.input) {
        st ^= st << 13;
        st ^= st >> 17;
        st ^= st << 5;
        x = (float)(st >> 8) / 8388608.0f - 1.0f;
    }

    const uint32_t nconv = aexrt_yolo_conv_plan_count(t.model);
    std::vector<AexrtConvPlanInfo> plan(nconv);
    for (uint32_t i = 0; i < nconv; ++i) {
        plan[i].struct_size = sizeof(AexrtConvPlanInfo);
        if (!aexrt_yolo_conv_plan_info(t.model, i, &plan[i])) {
            std::fprintf(stderr, "conv plan info %u failed\n", i);
            return 2;
        }
    }
    std::map<Shape, size_t> first;
    std::vector<Row> rows;
    for (const AexrtConvPlanInfo& p : plan)
        if (first.emplace(shape_of(p), rows.size()).second) {
            Row r;
            r.info = p;
            r.best = p.current_algorithm;
            rows.push_back(r);
        }
    if (limit && rows.size() > limit) rows.resize(limit);
    std::printf("convs %u, distinct shapes %zu\n", nconv, rows.size());

    std::vector<AexrtYoloDetection> base;
    std::vector<double> samples;
    for (uint32_t i = 0; i < t.warmup + t.runs; ++i) {
        const double ms = t.run(base);
        if (t.failed) {
            std::fprintf(stderr, "baseline run failed: %s\n", aexrt_yolo_get_last_error(t.model));
            return 2;
        }
        if (i >= t.warmup) samples.push_back(ms);
    }
    const double base_ms = median(samples);
    std::printf("baseline %.3f ms/run, %zu detections\n", base_ms, base.size());

    for (Row& r : rows) {
        const uint32_t cmd = r.info.command_index;
        if (r.info.in_fusion_group) {
            // a conv whose output feeds a fused residual add keeps its plan
            std::printf("  %s: fused, keeps alg %u\n", shape_str(r.info).c_str(), r.info.current_algorithm);
            continue;
        }
        r.current_ms = t.timed_step(cmd);
        for (uint32_t c = 0; c < r.info.candidate_count; ++c) {
            Candidate cd;
            cd.algorithm = r.info.candidates[c];
            if (cd.algorithm == r.info.current_algorithm) continue;
            if (aexrt_yolo_override_conv_algorithm(t.model, cmd, cd.algorithm)) {
                std::vector<AexrtYoloDetection> d;
                cd.ran = t.run(d) >= 0;
                cd.gate = cd.ran && same_detections(d, base);
                if (cd.gate) cd.ms = t.timed_step(cmd);
            }
            aexrt_yolo_override_conv_algorithm(t.model, cmd, r.info.current_algorithm);
            r.cands.push_back(cd);
        }
        r.best_ms = r.current_ms;
        for (const Candidate& cd : r.cands)
            if (cd.gate && cd.ms >= 0 && r.current_ms > 0 && cd.ms < 0.95 * r.current_ms &&
                (r.best == r.info.current_algorithm || cd.ms < r.best_ms)) {
                r.best = cd.algorithm;
                r.best_ms = cd.ms;
            }
        std::printf("  %s: alg %u %.4f ms -> alg %u %.4f ms\n", shape_str(r.info).c_str(), r.info.current_algorithm,
                    r.current_ms, r.best, r.best_ms);
    }

    // every command of a winning shape takes the winner
    std::vector<std::pair<uint32_t, uint32_t>> winners;
    for (const AexrtConvPlanInfo& p : plan) {
        auto it = first.find(shape_of(p));
        if (it == first.end() || it->second >= rows.size() || p.in_fusion_group) continue;
        const Row& r = rows[it->second];
        if (r.best != p.current_algorithm) winners.emplace_back(p.command_index, r.best);
    }
    const std::vector<std::pair<uint32_t, uint32_t>> all_winners = winners;
    auto apply = [&]() {
        for (const AexrtConvPlanInfo& p : plan)
            if (!p.in_fusion_group) aexrt_yolo_override_conv_algorithm(t.model, p.command_index, p.current_algorithm);
        for (const auto& w : winners) aexrt_yolo_override_conv_algorithm(t.model, w.first, w.second);
    };
    auto combo_ok = [&]() {
        std::vector<AexrtYoloDetection> d;
        for (uint32_t i = 0; i < t.warmup + 2; ++i)
            if (t.run(d) < 0) return false;
        return same_detections(d, base);
    };
    apply();
    while (!winners.empty() && !combo_ok()) {
        std::fprintf(stderr, "combination fails; dropping cmd#%u alg %u\n", winners.back().first,
                     winners.back().second);
        winners.pop_back();
        apply();
    }
    std::vector<AexrtYoloDetection> tuned;
    samples.clear();
    for (uint32_t i = 0; i < t.warmup + t.runs; ++i) {
        const double ms = t.run(tuned);
        if (i >= t.warmup && ms >= 0) samples.push_back(ms);
    }
    const double tuned_ms = median(samples);
    const bool gate = !t.failed && same_detections(tuned, base);
    std::printf("tuned %.3f ms/run (baseline %.3f), %zu overrides, final gate %s\n", tuned_ms, base_ms,
                winners.size(), gate ? "PASS" : "FAIL");

    std::ofstream rep(out_path, std::ios::binary);
    rep << "# conv_autotune report\n\n- engine: " << engine << "\n- device: " << device_index
        << "\n- distinct conv shapes: " << rows.size() << ", overrides applied: " << winners.size()
        << "\n- per-run time (profiled, steps launched one by one): baseline " << base_ms << " ms, tuned "
        << tuned_ms << " ms\n- final detection gate: " << (gate ? "PASS" : "FAIL") << "\n\n"
        << "| shape | planned alg | best alg | planned ms | best ms | failed the gate |\n|---|---|---|---|---|---|\n";
    for (const Row& r : rows) {
        std::string blocked;
        for (const Candidate& cd : r.cands)
            if (!cd.gate) blocked += std::to_string(cd.algorithm) + " ";
        rep << "| " << shape_str(r.info) << " | " << r.info.current_algorithm << " | " << r.best << " | "
            << r.current_ms << " | " << r.best_ms << " | " << blocked << " |\n";
    }
    if (!map_path.empty()) {
        // every single-shape winner (each passed the gate on its own): the
        // compiler rebuilds the whole plan around them
        std::ofstream m(map_path, std::ios::binary);
        m << "{\n";
        for (size_t i = 0; i < all_winners.size(); ++i)
            m << "    \"" << all_winners[i].first << "\": " << all_winners[i].second
              << (i + 1 < all_winners.size() ? ",\n" : "\n");
        m << "}\n";
    }
    if (!header_path.empty()) {
        std::ofstream h(header_path, std::ios::binary);
        h << "/* conv_autotune output for " << engine << ": after loading the engine, call\n"
          << " * aexrt_yolo_override_conv_algorithm(model, e.command_index, e.algorithm) for each entry. */\n"
          << "typedef struct AexrtTunedConvEntry {\n    unsigned command_index;\n    unsigned algorithm;\n"
          << "} AexrtTunedConvEntry;\n\nstatic const AexrtTunedConvEntry kAexrtTunedConvs[] = {\n";
        for (const auto& w : winners) h << "    {" << w.first << "u, " << w.second << "u},\n";
        if (winners.empty()) h << "    {0u, 0u},\n";
        h << "};\nstatic const unsigned kAexrtTunedConvCount = " << winners.size() << "u;\n";
    }
    aexrt_yolo_destroy(t.model);
    aexrt_hip_destroy_device(t.dev);
    return gate ? 0 : 3;
}
