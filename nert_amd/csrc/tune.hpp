#pragma once
// Per-geometry choice among kernel configurations, made by timing or read
// from a committed table.
//
// Which tile shape and split-K count is fastest depends on how a problem's
// tile count falls against the 256 CUs, which no simple rule captures across
// shapes. A choice fixes the order in which a geometry's sums are formed, so
// it also fixes the rounding: to make results reproducible across processes
// and machines, choices come first from a table (one line per geometry,
// nert_amd/tuning/gfx950.tsv next to the library, or the file that
// NERT_HIP_TUNE_TABLE names). A geometry the table lacks is timed on its
// first eager call: every candidate that fits runs on a scratch output (one
// warm-up launch, then ten launches captured into a HIP graph and replayed
// between HIP events on the caller's stream, as a replayed program runs
// them); the four fastest are timed again (three interleaved rounds) since the
// leaders are often closer than one pass's noise, and the fastest is kept
// for the rest of the process. NERT_HIP_TUNE_RECORD=<file> appends
// each such timed choice to <file> in the table's format, with the
// finalists' times after a '#'. A first call
// under stream capture cannot time anything and fixes the fallback instead,
// as does NERT_HIP_CONV_TUNE=0 in the environment.
//
// Table line: <family> <candidate count> <key integers, comma separated>
// <choice>; '#' starts a comment. A line whose family or candidate count no
// longer matches the caller is ignored, so a changed candidate list falls
// back to timing rather than to a wrong index.

#include "common.hpp"

#include <dlfcn.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace nert_hip {

// NERT_HIP_TUNE_LOG=1: print every candidate's time and the choice to stderr.
inline bool TuneLogEnabled() {
    static const bool enabled = [] {
        const char* e = std::getenv("NERT_HIP_TUNE_LOG");
        return e != nullptr && std::string(e) == "1";
    }();
    return enabled;
}

inline bool TuningEnabled() {
    static const bool enabled = [] {
        const char* e = std::getenv("NERT_HIP_CONV_TUNE");
        return e == nullptr || std::string(e) != "0";
    }();
    return enabled;
}

template <class Key>
std::string TableKey(const char* family, int count, const Key& key) {
    std::string s = std::string(family) + " " + std::to_string(count) + " ";
    for (size_t i = 0; i < key.size(); ++i) {
        s += (i != 0 ? "," : "") + std::to_string(key[i]);
    }
    return s;
}

// The committed choices: <dir of libnert_hip.so>/../tuning/gfx950.tsv, or
// $NERT_HIP_TUNE_TABLE. Read once; a missing file is an empty table.
inline const std::unordered_map<std::string, int>& TuneTable() {
    static const std::unordered_map<std::string, int> table = [] {
        std::unordered_map<std::string, int> t;
        std::string path;
        if (const char* e = std::getenv("NERT_HIP_TUNE_TABLE")) {
            path = e;
        } else {
            Dl_info info{};
            if (dladdr(reinterpret_cast<const void*>(&TuneLogEnabled), &info) != 0 && info.dli_fname != nullptr) {
                std::string lib = info.dli_fname;
                const size_t slash = lib.rfind('/');
                path = (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/../tuning/gfx950.tsv";
            }
        }
        std::ifstream in(path);
        std::string line;
        while (std::getline(in, line)) {
            const size_t hash = line.find('#');
            if (hash != std::string::npos) {
                line.resize(hash);
            }
            std::istringstream fields(line);
            std::string family, count, key;
            int choice = -1;
            if (fields >> family >> count >> key >> choice && choice >= 0) {
                t[family + " " + count + " " + key] = choice;
            }
        }
        return t;
    }();
    return table;
}

// Appends "<key> <choice> # <candidate>:<us> ..." (the finalists' re-timed
// microseconds after the '#', which table readers skip).
inline void RecordChoice(const std::string& table_key, int choice,
                         const std::vector<std::pair<int, float>>& finalists) {
    const char* path = std::getenv("NERT_HIP_TUNE_RECORD");
    if (path == nullptr || *path == 0) {
        return;
    }
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (FILE* f = std::fopen(path, "a")) {
        std::fprintf(f, "%s %d #", table_key.c_str(), choice);
        for (const auto& c : finalists) {
            std::fprintf(f, " %d:%.3f", c.first, c.second);
        }
        std::fprintf(f, "\n");
        std::fclose(f);
    }
}

// launch(i, scratch_y) -> false when candidate i does not fit; it must write
// its output to scratch_y (scratch_bytes long) instead of the caller's.
template <class Key, class Launch>
int ChooseConfig(const char* family, std::map<Key, int>& cache, std::mutex& mu, const Key& key,
                 size_t scratch_bytes, hipStream_t stream, int count, int fallback, Launch launch) {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
        return it->second;
    }
    const std::string table_key = TableKey(family, count, key);
    const auto& table = TuneTable();
    const auto row = table.find(table_key);
    if (row != table.end() && row->second < count) {
        if (TuneLogEnabled()) {
            std::fprintf(stderr, "nert_hip tune: table %s -> %d\n", table_key.c_str(), row->second);
        }
        cache.emplace(key, row->second);
        return row->second;
    }
    int best = fallback;
    bool timed = false;
    std::vector<std::pair<int, float>> finalist_us;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    Check(hipStreamIsCapturing(stream, &capture), "hipStreamIsCapturing");
    if (TuningEnabled() && capture == hipStreamCaptureStatusNone && count > 1 && scratch_bytes > 0) {
        timed = true;
        float* scratch = nullptr;
        Check(hipMalloc(&scratch, scratch_bytes), "hipMalloc(tuning output)");
        hipEvent_t start = nullptr, stop = nullptr;
        try {
            Check(hipEventCreate(&start), "hipEventCreate");
            Check(hipEventCreate(&stop), "hipEventCreate");
            // A candidate's time is measured as a replayed graph sees it:
            // `reps` back-to-back launches captured into one HIP graph, one
            // warm replay, then one replay between events. Timing eager
            // launches instead would count the host's launch gaps, which on
            // kernels of a few microseconds outweigh the kernels' own
            // differences. (The candidate's eager launch before its first
            // timing has grown every workspace it uses, so nothing allocates
            // under capture; the launches queue no memsets.)
            auto time_us = [&](int i, int reps) {
                Check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
                hipGraph_t graph = nullptr;
                try {
                    for (int r = 0; r < reps; ++r) {
                        launch(i, scratch);
                    }
                } catch (...) {
                    (void)hipStreamEndCapture(stream, &graph);
                    if (graph != nullptr) {
                        (void)hipGraphDestroy(graph);
                    }
                    throw;
                }
                Check(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
                hipGraphExec_t exec = nullptr;
                const hipError_t made = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
                (void)hipGraphDestroy(graph);
                Check(made, "hipGraphInstantiate(tuning)");
                float ms = 0.0f;
                try {
                    Check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
                    Check(hipEventRecord(start, stream), "hipEventRecord");
                    Check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
                    Check(hipEventRecord(stop, stream), "hipEventRecord");
                    Check(hipEventSynchronize(stop), "hipEventSynchronize");
                    Check(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
                } catch (...) {
                    (void)hipStreamSynchronize(stream);
                    (void)hipGraphExecDestroy(exec);
                    throw;
                }
                Check(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
                return ms * 1000.0f / static_cast<float>(reps);
            };
            // First pass: one warm eager launch, then a graph of ten launches.
            std::vector<std::pair<float, int>> first;
            for (int i = 0; i < count; ++i) {
                if (!launch(i, scratch)) {
                    continue;
                }
                const float us = time_us(i, 10);
                if (TuneLogEnabled()) {
                    std::fprintf(stderr, "nert_hip tune: candidate %d %.1f us\n", i, us);
                }
                first.emplace_back(us, i);
            }
            // The leaders are often within a few percent of each other, about
            // the first pass's noise: re-time the best four in three
            // interleaved rounds of ten launches and keep each one's fastest
            // round.
            std::sort(first.begin(), first.end());
            const size_t finalists = std::min<size_t>(first.size(), 4);
            std::vector<float> best_us(finalists, -1.0f);
            for (int round = 0; round < 3 && finalists > 1; ++round) {
                for (size_t f = 0; f < finalists; ++f) {
                    const float us = time_us(first[f].second, 10);
                    if (best_us[f] < 0.0f || us < best_us[f]) {
                        best_us[f] = us;
                    }
                }
            }
            for (size_t f = 0; f < finalists; ++f) {
                finalist_us.emplace_back(first[f].second, finalists > 1 ? best_us[f] : first[f].first);
            }
            if (!first.empty()) {
                best = first[0].second;
                float best_time = best_us[0];
                for (size_t f = 1; f < finalists; ++f) {
                    if (best_us[f] < best_time) {
                        best_time = best_us[f];
                        best = first[f].second;
                    }
                }
            }
        } catch (...) {
            (void)hipStreamSynchronize(stream);
            (void)hipEventDestroy(start);
            (void)hipEventDestroy(stop);
            (void)hipFree(scratch);
            throw;
        }
        Check(hipStreamSynchronize(stream), "hipStreamSynchronize");
        Check(hipEventDestroy(start), "hipEventDestroy");
        Check(hipEventDestroy(stop), "hipEventDestroy");
        Check(hipFree(scratch), "hipFree(tuning output)");
    }
    if (TuneLogEnabled()) {
        std::fprintf(stderr, "nert_hip tune: chose %d of %d for %s\n", best, count, table_key.c_str());
    }
    if (timed) {
        RecordChoice(table_key, best, finalist_us);
    }
    cache.emplace(key, best);
    return best;
}

} // namespace nert_hip
