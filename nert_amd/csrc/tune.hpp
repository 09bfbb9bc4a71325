#pragma once
// Per-geometry choice among kernel configurations, made by timing.
//
// Which tile shape and split-K count is fastest depends on how a problem's
// tile count falls against the 256 CUs, which no simple rule captures across
// shapes. So the first eager call of each geometry runs every candidate that
// fits on a scratch output (one warm-up and three timed launches each, HIP
// events on the caller's stream) and keeps the fastest; later calls of the
// geometry reuse it, so within a process a geometry is always computed the
// same way. The four fastest of that pass are timed again (two interleaved
// rounds of five launches) before the choice, since the leaders are often
// closer than one pass's noise. A first call under stream capture cannot time anything and fixes
// the fallback instead, as does NERT_HIP_CONV_TUNE=0 in the environment.

#include "common.hpp"

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
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

// launch(i, scratch_y) -> false when candidate i does not fit; it must write
// its output to scratch_y (scratch_bytes long) instead of the caller's.
template <class Key, class Launch>
int ChooseConfig(std::map<Key, int>& cache, std::mutex& mu, const Key& key, size_t scratch_bytes,
                 hipStream_t stream, int count, int fallback, Launch launch) {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
        return it->second;
    }
    int best = fallback;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    Check(hipStreamIsCapturing(stream, &capture), "hipStreamIsCapturing");
    if (TuningEnabled() && capture == hipStreamCaptureStatusNone && count > 1 && scratch_bytes > 0) {
        float* scratch = nullptr;
        Check(hipMalloc(&scratch, scratch_bytes), "hipMalloc(tuning output)");
        hipEvent_t start = nullptr, stop = nullptr;
        try {
            Check(hipEventCreate(&start), "hipEventCreate");
            Check(hipEventCreate(&stop), "hipEventCreate");
            auto time_us = [&](int i, int reps) {
                Check(hipEventRecord(start, stream), "hipEventRecord");
                for (int r = 0; r < reps; ++r) {
                    launch(i, scratch);
                }
                Check(hipEventRecord(stop, stream), "hipEventRecord");
                Check(hipEventSynchronize(stop), "hipEventSynchronize");
                float ms = 0.0f;
                Check(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
                return ms * 1000.0f / static_cast<float>(reps);
            };
            // First pass: one warm launch and three timed launches each.
            std::vector<std::pair<float, int>> first;
            for (int i = 0; i < count; ++i) {
                if (!launch(i, scratch)) {
                    continue;
                }
                const float us = time_us(i, 3);
                if (TuneLogEnabled()) {
                    std::fprintf(stderr, "nert_hip tune: candidate %d %.1f us\n", i, us);
                }
                first.emplace_back(us, i);
            }
            // The leaders are often within a few percent of each other, about
            // the first pass's noise: re-time the best four in two interleaved
            // rounds of five launches and keep each one's faster round.
            std::sort(first.begin(), first.end());
            const size_t finalists = std::min<size_t>(first.size(), 4);
            std::vector<float> best_us(finalists, -1.0f);
            for (int round = 0; round < 2 && finalists > 1; ++round) {
                for (size_t f = 0; f < finalists; ++f) {
                    const float us = time_us(first[f].second, 5);
                    if (best_us[f] < 0.0f || us < best_us[f]) {
                        best_us[f] = us;
                    }
                }
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
        std::fprintf(stderr, "nert_hip tune: chose %d of %d\n", best, count);
    }
    cache.emplace(key, best);
    return best;
}

} // namespace nert_hip
