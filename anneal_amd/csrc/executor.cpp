// executor.cpp — backend.Executor / SymbolicExecutor / Benchmarker mirror over ExecItem-shaped input,
// and the persistent plans that replay an item list as a HIP graph (tensor.JIT).
//
// Follows the reference's Run contract (backend/webgpu/executor.go:26-237, :576-922):
//   - bufs[0] is the output, bufs[1..] inputs in PARAM order;
//   - outputs with slot >= 0 share one allocation per slot sized for the largest user (4 bytes/element);
//   - final outputs are outputs no item reads; they are downloaded widened to f32 and keyed by uop_idx;
//   - inputs whose uop_idx is not in the schedule are ignored;
//   - every buffer a Run sees starts at zero, as freshly created WebGPU buffers do: a leaf with no input,
//     or an input shorter than its buffer, leaves zeros behind it;
//   - ah_run / ah_run_symbolic release every device object made for the call before returning.
// Differences by design: kernels come from hiprtc-compiled HIP source (cached per source for the device
// lifetime instead of recompiled each Run) or from "tmpl:" keys naming hand-written kernels, which may
// also write later PARAMs ("side outputs"); a side output no item reads is returned as a final output too.
//
// A plan (ah_plan_*) is the same Run kept alive: its item list is copied, its kernels resolved and its
// buffers allocated once (re-sized when a larger symbolic binding arrives), and with AH_PLAN_GRAPH each
// binding's kernel sequence is captured once as a HIP graph and replayed on later runs. This is the device
// half of tensor.JIT (tensor/jit.go:178-215), which replays one captured item list through Run/RunSymbolic
// with fresh leaf data on every step.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>

#include "ah_internal.h"
#include "itemops.h"

namespace {

int64_t bound_size(int64_t size, const std::vector<int64_t> &shape, int64_t n) {
    if (size > 0) return size;
    if (shape.empty()) return size;
    int64_t s = 1;
    for (int64_t d : shape) s *= (d == 0 ? n : d);
    return s;
}

}  // namespace

struct ah_plan {
    struct Buf {
        uint32_t uop;
        int64_t size;
        int32_t dtype;
        int32_t slot;
        std::vector<int64_t> shape;
        int64_t elems(int64_t n) const { return bound_size(size, shape, n); }
    };
    struct Item {
        std::string source;
        std::vector<Buf> bufs;
        int n_sym = 0;
        int32_t ls[3], wg[3];
        ah_kernel *k = nullptr;
        std::vector<int> writes;   // PARAM positions written: 0 plus the template's side outputs
        std::vector<bool> clear;   // per entry of writes: zero before the launch
    };
    // One device buffer per uop_idx (slot outputs share their slot's allocation).
    struct Mem {
        int32_t dtype = AH_F32;
        int slot = -1;
        bool leaf = true;          // not written by any item: filled from the inputs
        std::vector<const Buf *> descs;
        void *ptr = nullptr;
        int64_t elems(int64_t n) const {
            int64_t e = 0;
            for (const Buf *b : descs) e = std::max(e, b->elems(n));
            return e;
        }
    };

    ah_device *dev = nullptr;
    std::vector<Item> items;
    bool has_sym = false;
    std::string symvar;            // SymVars[0] of the first symbolic item (executor.go:817-822)
    std::map<uint32_t, Mem> mem;
    std::vector<uint32_t> finals;  // final outputs in item order
    std::vector<void *> owned;
    int64_t alloc_n = -1;          // binding the allocations are sized for
    std::map<int64_t, ah_graph *> graphs;
    int64_t captures = 0, replays = 0;

    ~ah_plan() {
        if (dev) hipStreamSynchronize(dev->stream);
        drop_graphs();
        release();
    }
    void drop_graphs() {
        for (auto &kv : graphs) ah_graph_destroy(kv.second);
        graphs.clear();
    }
    void release() {
        for (void *p : owned) hipFree(p);
        owned.clear();
        for (auto &kv : mem) kv.second.ptr = nullptr;
    }
};

namespace ah {
namespace {

int plan_build(ah_device *d, const ah_exec_item *items, int32_t n_items, ah_plan *p) {
    p->dev = d;
    p->items.resize(n_items);
    for (int i = 0; i < n_items; i++) {
        const ah_exec_item &src = items[i];
        if (src.n_bufs < 1 || !src.bufs || !src.source)
            return set_error(AH_ERR_INVALID, "ah_run: kernel %d has no buffers or source", i);
        ah_plan::Item &it = p->items[i];
        it.source = src.source;
        for (int j = 0; j < src.n_bufs; j++) {
            const ah_buffer_desc &b = src.bufs[j];
            ah_plan::Buf c{b.uop_idx, b.size, b.dtype, b.slot, {}};
            if (b.shape && b.rank > 0) c.shape.assign(b.shape, b.shape + b.rank);
            if (dtype_bytes(b.dtype) <= 0) return set_error(AH_ERR_UNSUPPORTED, "ah_run: kernel %d: dtype %d", i, b.dtype);
            it.bufs.push_back(c);
        }
        it.n_sym = src.n_sym_vars > 0 && src.sym_vars ? src.n_sym_vars : 0;
        if (it.n_sym && !p->has_sym) {
            p->has_sym = true;
            p->symvar = src.sym_vars[0] ? src.sym_vars[0] : "";
        }
        for (int a = 0; a < 3; a++) {
            it.ls[a] = std::max(1, src.local_size[a]);
            it.wg[a] = std::max(1, src.workgroup_count[a]);
        }
        int rc = ah_module_get(d, it.source.c_str(), "kernel", &it.k);
        if (rc) return set_error(rc, "ah_run: kernel %d: %s", i, ah_last_error());
        // Writes: data0 always; a template's side outputs too. Only templates are known to overwrite
        // every element of data0, so other kernels' outputs are cleared before they run.
        it.writes.push_back(0);
        it.clear.push_back(it.k->tmpl == nullptr);
        if (it.k->tmpl)
            for (auto &s : it.k->tmpl->side) {
                if (s.param >= (int)it.bufs.size())
                    return set_error(AH_ERR_INVALID, "ah_run: kernel %d: %s writes PARAM %d of %zu", i,
                                     it.k->tmpl->name.c_str(), s.param, it.bufs.size());
                it.writes.push_back(s.param);
                it.clear.push_back(s.zero);
            }
    }
    // buffer table
    std::set<uint32_t> read_any;
    for (auto &it : p->items) {
        for (size_t j = 0; j < it.bufs.size(); j++) {
            ah_plan::Mem &m = p->mem[it.bufs[j].uop];
            m.descs.push_back(&it.bufs[j]);
            m.dtype = it.bufs[j].dtype;
        }
        for (int w : it.writes) {
            ah_plan::Mem &m = p->mem[it.bufs[w].uop];
            m.leaf = false;
            m.dtype = it.bufs[w].dtype;
            if (w == 0 && it.bufs[0].slot >= 0) m.slot = it.bufs[0].slot;
        }
    }
    for (auto &it : p->items)
        for (size_t j = 1; j < it.bufs.size(); j++) {
            bool written_here = std::find(it.writes.begin(), it.writes.end(), (int)j) != it.writes.end();
            if (!written_here) read_any.insert(it.bufs[j].uop);
        }
    for (auto &it : p->items)
        for (int w : it.writes) {
            uint32_t u = it.bufs[w].uop;
            if (!read_any.count(u) && std::find(p->finals.begin(), p->finals.end(), u) == p->finals.end())
                p->finals.push_back(u);
        }
    return AH_OK;
}

// Allocates every buffer for binding n (once, or again when n outgrows the allocation) and zeroes it.
int plan_alloc(ah_plan *p, int64_t n) {
    if (p->alloc_n >= 0 && (!p->has_sym || n <= p->alloc_n)) return AH_OK;
    AH_HIP(hipStreamSynchronize(p->dev->stream));
    p->drop_graphs();
    p->release();
    std::map<int, int64_t> slot_bytes;
    for (auto &kv : p->mem)
        if (kv.second.slot >= 0)
            slot_bytes[kv.second.slot] = std::max(slot_bytes[kv.second.slot], std::max<int64_t>(kv.second.elems(n), 1) * 4);
    std::map<int, void *> slot_ptr;
    auto alloc = [&](int64_t bytes, void **out) -> int {
        bytes = std::max<int64_t>(bytes, 4);
        AH_HIP(hipMalloc(out, (size_t)bytes));
        p->owned.push_back(*out);
        AH_HIP(zero_fill(*out, bytes, p->dev->stream));
        return AH_OK;
    };
    for (auto &kv : slot_bytes)
        if (int rc = alloc(kv.second, &slot_ptr[kv.first])) return rc;
    for (auto &kv : p->mem) {
        ah_plan::Mem &m = kv.second;
        if (m.slot >= 0) m.ptr = slot_ptr[m.slot];
        else if (int rc = alloc(m.elems(n) * dtype_bytes(m.dtype), &m.ptr)) return rc;
    }
    p->alloc_n = p->has_sym ? n : 0;
    return AH_OK;
}

// Enqueues the item list: clears, then each kernel with its buffers.
int plan_enqueue(ah_plan *p, int64_t n, bool symbolic) {
    ah_device *d = p->dev;
    for (size_t i = 0; i < p->items.size(); i++) {
        ah_plan::Item &it = p->items[i];
        for (size_t w = 0; w < it.writes.size(); w++) {
            if (!it.clear[w]) continue;
            const ah_plan::Mem &m = p->mem[it.bufs[it.writes[w]].uop];
            int64_t bytes = m.elems(n) * dtype_bytes(m.dtype);
            if (m.slot >= 0) bytes = std::max<int64_t>(m.elems(n), 1) * 4;
            AH_HIP(zero_fill(m.ptr, bytes, d->stream));
        }
        std::vector<void *> ptrs;
        for (auto &b : it.bufs) ptrs.push_back(p->mem[b.uop].ptr);
        std::vector<int32_t> sc;
        if (symbolic && it.n_sym > 0) sc.assign(4, (int32_t)n);   // params_n: a 16-byte uniform
        uint32_t grid[3], block[3];
        for (int a = 0; a < 3; a++) {
            grid[a] = (uint32_t)it.wg[a];
            block[a] = (uint32_t)it.ls[a];
        }
        if (symbolic && it.n_sym > 0) {   // 1-D dispatch over the bound output (executor.go:874-898)
            int64_t out_elems = it.bufs[0].elems(n);
            grid[0] = (uint32_t)std::max<int64_t>(1, (out_elems + block[0] - 1) / block[0]);
        }
        int rc = ah_launch(d, it.k, grid, block, ptrs.data(), (int32_t)ptrs.size(), sc.data(), (int32_t)sc.size());
        if (rc) return set_error(rc, "ah_run: kernel %zu: %s", i, ah_last_error());
    }
    return AH_OK;
}

int plan_run(ah_plan *p, const ah_input *inputs, int32_t n_inputs, int64_t n, bool symbolic, bool graph,
             ah_output **outputs, int32_t *n_outputs) {
    ah_device *d = p->dev;
    *outputs = nullptr;
    *n_outputs = 0;
    if (p->items.empty()) return AH_OK;
    if (int rc = plan_alloc(p, n)) return rc;
    // Template workspaces for this binding; a workspace that moves invalidates captured graphs. First,
    // every buffer a template reads or writes must hold what its key's shape needs: the hand-written
    // kernels index by the key's M, N, K (and the like), not by the buffer sizes.
    for (size_t i = 0; i < p->items.size(); i++) {
        const ah_plan::Item &it = p->items[i];
        TemplateKernel *t = it.k->tmpl;
        if (!t || !t->bytes) continue;
        const std::vector<int64_t> want = t->bytes(symbolic ? n : 0);
        if (want.size() > it.bufs.size())
            return set_error(AH_ERR_INVALID, "ah_run: kernel %zu (%s) takes %zu buffers, got %zu", i, t->name.c_str(),
                             want.size(), it.bufs.size());
        for (size_t j = 0; j < want.size(); j++) {
            const ah_plan::Mem &m = p->mem[it.bufs[j].uop];
            const int64_t have = m.slot >= 0 ? std::max<int64_t>(m.elems(n), 1) * 4 : m.elems(n) * dtype_bytes(m.dtype);
            if (want[j] > have)
                return set_error(AH_ERR_INVALID, "ah_run: kernel %zu (%s): PARAM %zu (uop %u) holds %lld bytes, the key's "
                                 "shape needs %lld", i, t->name.c_str(), j, it.bufs[j].uop, (long long)have, (long long)want[j]);
        }
    }
    for (size_t i = 0; i < p->items.size(); i++) {
        TemplateKernel *t = p->items[i].k->tmpl;
        if (!t) continue;
        void *before = t->ws;
        if (int rc = template_prepare(t, symbolic ? n : 0)) return set_error(rc, "ah_run: kernel %zu: %s", i, ah_last_error());
        if (t->ws != before) p->drop_graphs();
    }
    // Leaves: the input's elements, zeros after them (fresh-buffer semantics); no input: all zeros.
    std::map<uint32_t, const ah_input *> in;
    for (int i = 0; i < n_inputs; i++) in[inputs[i].uop_idx] = &inputs[i];
    for (auto &kv : p->mem) {
        ah_plan::Mem &m = kv.second;
        if (!m.leaf) continue;
        const int64_t elems = m.elems(n);
        auto f = in.find(kv.first);
        const int64_t k = f == in.end() ? 0 : std::min<int64_t>(f->second->n, elems);
        if (k < elems) AH_HIP(zero_fill(m.ptr, std::max<int64_t>(elems, 1) * dtype_bytes(m.dtype), d->stream));
        if (k > 0) {
            if (!f->second->data) return set_error(AH_ERR_INVALID, "ah_run: input %u has no data", kv.first);
            if (int rc = ah_upload(d, m.ptr, f->second->data, k, m.dtype)) return rc;
        }
    }
    const int64_t key = symbolic ? n : 0;
    if (graph) {
        auto g = p->graphs.find(key);
        if (g == p->graphs.end()) {
            if (int rc = ah_graph_begin(d)) return rc;
            int rc = plan_enqueue(p, n, symbolic);
            ah_graph *cg = nullptr;
            int rc2 = ah_graph_end(d, &cg);
            if (rc) { ah_graph_destroy(cg); return rc; }
            if (rc2) return rc2;
            g = p->graphs.emplace(key, cg).first;
            p->captures++;
        } else {
            p->replays++;
        }
        if (int rc = ah_graph_replay(d, g->second)) return rc;
    } else if (int rc = plan_enqueue(p, n, symbolic)) {
        return rc;
    }
    // Final outputs, widened to f32 (ah_download applies the codec).
    std::vector<ah_output> outs;
    for (uint32_t u : p->finals) {
        const ah_plan::Mem &m = p->mem[u];
        ah_output r;
        r.uop_idx = u;
        r.n = m.elems(n);
        r.data = (float *)malloc((size_t)std::max<int64_t>(r.n, 1) * 4);
        int rc = r.data ? ah_download(d, r.data, m.ptr, r.n, m.dtype) : set_error(AH_ERR_NOMEM, "ah_run: output buffer");
        if (rc) {
            free(r.data);
            for (auto &x : outs) free(x.data);
            return rc;
        }
        outs.push_back(r);
    }
    AH_HIP(hipStreamSynchronize(d->stream));
    ah_output *arr = (ah_output *)malloc(sizeof(ah_output) * std::max<size_t>(outs.size(), 1));
    for (size_t i = 0; i < outs.size(); i++) arr[i] = outs[i];
    *outputs = arr;
    *n_outputs = (int32_t)outs.size();
    return AH_OK;
}

// Binding of the plan's symbolic variable; like the reference, only SymVars[0] of the first symbolic
// item is looked up (backend/webgpu/executor.go:817-822).
int find_binding(const ah_plan *p, const char *const *names, const int64_t *values, int32_t n_bind, int64_t *n) {
    *n = 0;
    if (!p->has_sym) return AH_OK;
    for (int b = 0; b < n_bind; b++)
        if (names && names[b] && values && p->symvar == names[b]) {
            if (values[b] < 0) return set_error(AH_ERR_INVALID, "binding %s = %lld is negative", names[b], (long long)values[b]);
            *n = values[b];
            return AH_OK;
        }
    return set_error(AH_ERR_INVALID, "no binding for %s", p->symvar.c_str());
}

}  // namespace
}  // namespace ah

using namespace ah;

extern "C" {

int ah_run(ah_device *d, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
           ah_output **outputs, int32_t *n_outputs) {
    if (!d || (!items && n_items) || (!inputs && n_inputs) || !outputs || !n_outputs)
        return set_error(AH_ERR_INVALID, "ah_run: null argument");
    ah_plan p;
    int rc = plan_build(d, items, n_items, &p);
    if (rc == AH_OK) rc = plan_run(&p, inputs, n_inputs, 0, false, false, outputs, n_outputs);
    return rc;
}

int ah_run_symbolic(ah_device *d, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
                    const char *const *bind_names, const int64_t *bind_values, int32_t n_bind, ah_output **outputs,
                    int32_t *n_outputs) {
    if (!d || (!items && n_items) || (!inputs && n_inputs) || !outputs || !n_outputs)
        return set_error(AH_ERR_INVALID, "ah_run_symbolic: null argument");
    ah_plan p;
    int rc = plan_build(d, items, n_items, &p);
    int64_t n = 0;
    if (rc == AH_OK) {
        rc = find_binding(&p, bind_names, bind_values, n_bind, &n);
        if (rc) rc = set_error(rc, "ah_run_symbolic: %s", ah_last_error());
    }
    if (rc == AH_OK) rc = plan_run(&p, inputs, n_inputs, n, true, false, outputs, n_outputs);
    return rc;
}

int ah_plan_create(ah_device *d, const ah_exec_item *items, int32_t n_items, ah_plan **out) {
    if (!d || (!items && n_items) || !out) return set_error(AH_ERR_INVALID, "ah_plan_create: null argument");
    ah_plan *p = new ah_plan();
    int rc = plan_build(d, items, n_items, p);
    if (rc) {
        delete p;
        return rc;
    }
    *out = p;
    return AH_OK;
}

int ah_plan_run(ah_plan *p, const ah_input *inputs, int32_t n_inputs, const char *const *bind_names,
                const int64_t *bind_values, int32_t n_bind, int32_t flags, ah_output **outputs, int32_t *n_outputs) {
    if (!p || (!inputs && n_inputs) || !outputs || !n_outputs) return set_error(AH_ERR_INVALID, "ah_plan_run: null argument");
    int64_t n = 0;
    if (int rc = find_binding(p, bind_names, bind_values, n_bind, &n)) return set_error(rc, "ah_plan_run: %s", ah_last_error());
    return plan_run(p, inputs, n_inputs, n, p->has_sym, (flags & AH_PLAN_GRAPH) != 0, outputs, n_outputs);
}

int ah_plan_stats(const ah_plan *p, int64_t *captures, int64_t *replays) {
    if (!p) return set_error(AH_ERR_INVALID, "ah_plan_stats: null plan");
    if (captures) *captures = p->captures;
    if (replays) *replays = p->replays;
    return AH_OK;
}

void ah_plan_destroy(ah_plan *p) { delete p; }

void ah_outputs_free(ah_output *outputs, int32_t n) {
    if (!outputs) return;
    for (int i = 0; i < n; i++) free(outputs[i].data);
    free(outputs);
}

int ah_benchmark(ah_device *d, const ah_exec_item *item, int32_t warmup, int32_t iterations, ah_bench_result *out) {
    if (!d || !item || !out) return set_error(AH_ERR_INVALID, "ah_benchmark: null argument");
    if (iterations <= 0) return set_error(AH_ERR_INVALID, "benchmark: iterations must be > 0");   // benchmark.go:29-31
    ah_kernel *k = nullptr;
    int rc = ah_module_get(d, item->source, "kernel", &k);
    if (rc) return rc;
    if (k->tmpl && (rc = template_prepare(k->tmpl, 0))) return rc;
    if (k->tmpl && k->tmpl->bytes) {   // buffers sized below what the key's shape needs: refuse before launching
        const std::vector<int64_t> want = k->tmpl->bytes(0);
        if ((int32_t)want.size() > item->n_bufs)
            return set_error(AH_ERR_INVALID, "benchmark: %s takes %zu buffers, got %d", k->tmpl->name.c_str(), want.size(), item->n_bufs);
        for (size_t j = 0; j < want.size(); j++)
            if (want[j] > std::max<int64_t>(item->bufs[j].size, 1) * dtype_bytes(item->bufs[j].dtype))
                return set_error(AH_ERR_INVALID, "benchmark: %s: PARAM %zu is smaller than the key's shape needs",
                                 k->tmpl->name.c_str(), j);
    }
    std::vector<void *> ptrs;
    auto release = [&]() { for (void *p : ptrs) hipFree(p); };
    for (int j = 0; j < item->n_bufs; j++) {
        void *p = nullptr;
        const size_t bytes = (size_t)std::max<int64_t>(item->bufs[j].size, 1) * dtype_bytes(item->bufs[j].dtype);
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) { release(); return fail_hip(e, "benchmark: hipMalloc"); }
        ptrs.push_back(p);
        e = zero_fill(p, (long)bytes, d->stream);
        if (e != hipSuccess) { release(); return fail_hip(e, "benchmark: zero fill"); }
    }
    uint32_t grid[3], block[3];
    for (int a = 0; a < 3; a++) {
        grid[a] = (uint32_t)std::max(1, item->workgroup_count[a]);
        block[a] = (uint32_t)std::max(1, item->local_size[a]);
    }
    hipEvent_t e0, e1;
    hipEventCreateWithFlags(&e0, hipEventDisableSystemFence);   // timing only
    hipEventCreateWithFlags(&e1, hipEventDisableSystemFence);
    std::vector<double> us;
    for (int i = 0; i < warmup + iterations && rc == AH_OK; i++) {
        hipEventRecord(e0, d->stream);
        rc = ah_launch(d, k, grid, block, ptrs.data(), (int32_t)ptrs.size(), nullptr, 0);
        hipEventRecord(e1, d->stream);
        if (rc == AH_OK && hipEventSynchronize(e1) != hipSuccess) rc = set_error(AH_ERR_HIP, "benchmark: sync failed");
        float ms = 0.0f;
        if (rc == AH_OK && i >= warmup) {
            hipEventElapsedTime(&ms, e0, e1);
            us.push_back(ms * 1000.0);
        }
    }
    hipStreamSynchronize(d->stream);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    release();
    if (rc) return rc;
    std::sort(us.begin(), us.end());
    double sum = 0, sq = 0;
    for (double v : us) sum += v;
    double mean = sum / us.size();
    for (double v : us) sq += (v - mean) * (v - mean);
    out->min_us = us.front();
    out->max_us = us.back();
    out->median_us = us[us.size() / 2];
    out->mean_us = mean;
    out->stddev_us = sqrt(sq / us.size());
    out->cv = mean > 0 ? out->stddev_us / mean : 0;
    return AH_OK;
}

}  // extern "C"
