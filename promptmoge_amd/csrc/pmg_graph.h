// Capture-once / replay cache of HIP graphs, keyed by the buffers and stream of an enqueue sequence.
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "pmg_common.h"

namespace pmg {

// A key is the sequence's kind tag, its buffers and the stream, padded with nullptr.
constexpr int kGraphKey = 12;

struct GraphCache {
    struct Entry {
        const void* key[kGraphKey];
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<Entry> entries;
    size_t max_entries = 4;

    // Destroys the cached graphs. A replay may still be running on the stream it was launched on, so the device is
    // synchronised first (this runs on eviction, new weights and destruction only).
    void clear() {
        if (entries.empty()) return;
        (void)hipDeviceSynchronize();
        for (auto& g : entries) {
            (void)hipGraphExecDestroy(g.exec);
            (void)hipGraphDestroy(g.graph);
        }
        entries.clear();
    }

    // Runs `enqueue` on `s`: captured into a graph the first time `key` is seen, replayed after. The legacy default
    // stream cannot be captured; on it (or with use_graph off) the work is enqueued eagerly.
    template <typename F>
    int run(const void* const (&key)[kGraphKey], hipStream_t s, bool use_graph, F&& enqueue) {
        if (!use_graph || s == nullptr) return enqueue();
        for (auto& g : entries)
            if (std::memcmp(g.key, key, sizeof key) == 0) {
                PMG_CHECK_HIP(hipGraphLaunch(g.exec, s));
                return PMG_OK;
            }
        if (entries.size() >= max_entries) clear();
        PMG_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        const int e = enqueue();
        hipGraph_t graph = nullptr;
        const hipError_t ce = hipStreamEndCapture(s, &graph);
        if (e) {
            if (graph) (void)hipGraphDestroy(graph);
            return e;
        }
        if (ce != hipSuccess) return fail(PMG_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ce));
        hipGraphExec_t exec = nullptr;
        const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (ie != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return fail(PMG_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(ie));
        }
        Entry g{};
        std::memcpy(g.key, key, sizeof key);
        g.graph = graph;
        g.exec = exec;
        entries.push_back(g);
        PMG_CHECK_HIP(hipGraphLaunch(exec, s));
        return PMG_OK;
    }
};

}  // namespace pmg
