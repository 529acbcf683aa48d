// Test harness (not product code): a worker pool in the shape of nnml's,
// driving the flash-attention binding the way the reference's scheduler
// drives an op.
//
// nnml runs a graph with nth worker threads that each walk the nodes in
// order, call the node's op with their own (ith, nth), and then meet at a
// global barrier before the next node (nnml_single_graph_compute_thread,
// nnml/src/scheduler.cpp:122-146; nnml_barrier_global, nnml/src/thread.cpp:
// 246-269: an arrival count and a pass count, spinning until the pass count
// moves). Here every worker calls al_fattn_f16_worker on each node.
//
// Two observations make the contract checkable from a test:
//   - workers other than 0 get a copy of each node whose dst is a canary
//     buffer (`others`); if any of them launched, its canary changes;
//   - right after the barrier that follows node i, the last worker asks the
//     node's stream whether all its work has finished (hipStreamQuery), which
//     holds only if worker 0 waited for the stream before the barrier.
#include <hip/hip_runtime.h>

#include <atomic>
#include <thread>
#include <vector>

#include "arclight_fattn.h"

namespace {

struct Barrier {
    std::atomic<int> arrived{0};
    std::atomic<int> passed{0};
    int total = 1;

    void wait() {
        if (total <= 1) return;
        const int p = passed.load(std::memory_order_relaxed);
        if (arrived.fetch_add(1, std::memory_order_seq_cst) == total - 1) {
            arrived.store(0, std::memory_order_relaxed);
            passed.fetch_add(1, std::memory_order_seq_cst);
            return;
        }
        while (passed.load(std::memory_order_relaxed) == p) std::this_thread::yield();
        std::atomic_thread_fence(std::memory_order_seq_cst);
    }
};

}  // namespace

// nodes[i]: node i as worker 0 sees it; others[i]: as workers 1..nth-1 see
// it. status[w * n_nodes + i]: worker w's return code on node i.
// done_after_barrier[i]: 1 if node i's stream had no pending work right
// after the barrier that follows it, 0 if it still had, -1 on a query error.
extern "C" int al_harness_run_workers(const al_fattn_args * nodes, const al_fattn_args * others, int n_nodes,
                                      int nth, int * status, int * done_after_barrier) {
    if (nth < 1 || n_nodes < 0) return -1;
    Barrier bar;
    bar.total = nth;
    auto work = [&](int ith) {
        for (int i = 0; i < n_nodes; ++i) {
            const al_fattn_args * node = ith == 0 ? &nodes[i] : &others[i];
            status[ith * n_nodes + i] = al_fattn_f16_worker(node, ith, nth);
            bar.wait();
            if (ith == nth - 1) {
                const hipError_t q = hipStreamQuery((hipStream_t) nodes[i].stream);
                done_after_barrier[i] = q == hipSuccess ? 1 : (q == hipErrorNotReady ? 0 : -1);
            }
            bar.wait();                                  // the query happens before the next node
        }
    };
    std::vector<std::thread> th;
    for (int w = 1; w < nth; ++w) th.emplace_back(work, w);
    work(0);
    for (auto & t : th) t.join();
    return 0;
}
