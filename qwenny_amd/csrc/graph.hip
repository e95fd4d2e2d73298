// Stream capture of product launches into replayable HIP graphs: the capture primitive under the reference engine's
// graph cache (Graphs::run, src/cuda/core.rs:1151-1192, which captures whole decode steps of n <= 32 tokens and
// replays them). The cache itself (keys, LRU, memory floor) stays with the caller. Every product entry point of this
// library is capture-safe: no allocation, no host synchronisation and no memset node (the kernels leave their
// counters and tables at zero themselves), so a captured sequence replays to the eager results.
#include <hip/hip_runtime.h>

#include <new>

#include "../../include/qwenny_hip.h"
#include "internal.h"

struct qh_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

using qh::fail;

extern "C" int qh_graph_begin(void* stream) {
    if (!stream) return fail(QH_EINVAL, "graph capture: the null stream cannot be captured");
    // thread-local mode: another thread's unrelated HIP calls are not part of this capture and do not invalidate it
    const hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(QH_EHIP, "graph capture: hipStreamBeginCapture: %s", hipGetErrorString(e));
    return QH_OK;
}

extern "C" int qh_graph_end(void* stream, qh_graph** out) {
    if (!stream || !out) return fail(QH_EINVAL, "graph capture end: null");
    *out = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e != hipSuccess || !g) return fail(QH_EHIP, "graph capture end: hipStreamEndCapture: %s", hipGetErrorString(e));
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(QH_EHIP, "graph capture end: hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    qh_graph* r = new (std::nothrow) qh_graph{g, x};
    if (!r) {
        (void)hipGraphExecDestroy(x);
        (void)hipGraphDestroy(g);
        return fail(QH_EINVAL, "graph capture end: out of host memory");
    }
    *out = r;
    return QH_OK;
}

extern "C" int qh_graph_launch(const qh_graph* g, void* stream) {
    if (!g) return fail(QH_EINVAL, "graph launch: null graph");
    const hipError_t e = hipGraphLaunch(g->exec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(QH_EHIP, "graph launch: %s", hipGetErrorString(e));
    return QH_OK;
}

extern "C" void qh_graph_free(qh_graph* g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
}
