// executor.cpp — backend.Executor / SymbolicExecutor / Benchmarker mirror over ExecItem-shaped input.
//
// Follows the reference's Run contract (backend/webgpu/executor.go:26-237, :576-922):
//   - bufs[0] is the output, bufs[1..] inputs in PARAM order;
//   - outputs with slot >= 0 share one allocation per slot sized for the largest user;
//   - final outputs are outputs no item reads; they are downloaded widened to f32 and keyed by uop_idx;
//   - inputs whose uop_idx is not in the schedule are ignored;
//   - every device object made for the call is released before returning.
// Differences by design: kernels come from hiprtc-compiled HIP source (cached per source for the device
// lifetime instead of recompiled each Run) or from "tmpl:" keys naming hand-written kernels.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>

#include "ah_internal.h"
#include "gemm.h"

namespace ah {

static std::unordered_map<std::string, std::string> parse_params(const std::string &s, std::string *name) {
    std::unordered_map<std::string, std::string> out;
    size_t p = s.find(';');
    *name = s.substr(5, p == std::string::npos ? std::string::npos : p - 5);
    while (p != std::string::npos) {
        size_t q = s.find(';', p + 1);
        std::string kv = s.substr(p + 1, q == std::string::npos ? std::string::npos : q - p - 1);
        size_t e = kv.find('=');
        if (e != std::string::npos) out[kv.substr(0, e)] = kv.substr(e + 1);
        p = q;
    }
    return out;
}

// "tmpl:gemm;dtype=f16;epi=bias_relu;ta=0;tb=0;M=4096;N=4096;K=1024[;variant=3]"
// PARAM order: data0 = C, data1 = A, data2 = B, data3 = bias (bias epilogues) or aux (mask).
// M may be "sym": it is then taken from the first symbolic scalar (the bound batch size).
int template_create(const std::string &source, TemplateKernel **out) {
    std::string name;
    auto params = parse_params(source, &name);
    auto geti = [&](const char *k, long dflt) -> long {
        auto it = params.find(k);
        return it == params.end() ? dflt : strtol(it->second.c_str(), nullptr, 10);
    };
    if (name == "gemm") {
        GemmDesc base;
        memset(&base, 0, sizeof base);
        std::string dt = params.count("dtype") ? params["dtype"] : "f32";
        if (dt != "f32" && dt != "f16") return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: dtype %s", dt.c_str());
        base.dtype = dt == "f16" ? GEMM_F16 : GEMM_F32;
        std::string epi = params.count("epi") ? params["epi"] : "store";
        static const std::map<std::string, int> epis = {{"store", EPI_STORE}, {"bias", EPI_BIAS},
                                                        {"bias_relu", EPI_BIAS_RELU}, {"mask", EPI_MASK}};
        auto ei = epis.find(epi);
        if (ei == epis.end()) return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: epilogue %s", epi.c_str());
        base.epi = ei->second;
        base.ta = (int)geti("ta", 0);
        base.tb = (int)geti("tb", 0);
        bool msym = params.count("M") && params["M"] == "sym";
        base.M = msym ? 0 : (int)geti("M", -1);
        base.N = (int)geti("N", -1);
        base.K = (int)geti("K", -1);
        base.scale = 1.0f;
        base.variant = (int)geti("variant", 0);
        if (base.variant < 0 || base.variant > kGemm16Variants) return set_error(AH_ERR_INVALID, "tmpl gemm: variant %d", base.variant);
        if ((!msym && base.M < 0) || base.N <= 0 || base.K < 0) return set_error(AH_ERR_INVALID, "tmpl gemm: M/N/K required");
        auto *t = new TemplateKernel();
        t->key = source;
        t->params = params;
        t->run = [base, msym](ah_device *d, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
            GemmDesc g = base;
            if (msym) {
                if (ns < 1) return set_error(AH_ERR_INVALID, "tmpl gemm: symbolic M needs a binding");
                g.M = sc[0];
            }
            int need = (g.epi == EPI_STORE) ? 3 : 4;
            if (n_ptrs < need) return set_error(AH_ERR_INVALID, "tmpl gemm: needs %d buffers, got %d", need, n_ptrs);
            g.C = ptrs[0];
            g.A = ptrs[1];
            g.B = ptrs[2];
            if (g.epi == EPI_BIAS || g.epi == EPI_BIAS_RELU) g.bias = ptrs[3];
            if (g.epi == EPI_MASK) { g.aux = ptrs[3]; g.ldaux = g.N; }
            g.lda = g.ta ? g.M : g.K;
            g.ldb = g.tb ? g.N : g.K;
            g.ldc = g.N;
            AH_HIP(gemm_launch(g, d->stream));
            return AH_OK;
        };
        *out = t;
        return AH_OK;
    }
    return set_error(AH_ERR_UNSUPPORTED, "unknown template '%s'", name.c_str());
}

// ── Run ─────────────────────────────────────────────────────────────────────

namespace {

struct RunState {
    ah_device *dev;
    std::vector<void *> owned;
    std::map<uint32_t, void *> ptr;
    std::map<uint32_t, int32_t> dtype;
    std::map<uint32_t, int64_t> elems;
    ~RunState() {
        for (void *p : owned) hipFree(p);
    }
};

int64_t bound_size(const ah_buffer_desc &b, int64_t n) {
    if (b.size > 0) return b.size;
    if (!b.shape || b.rank <= 0) return b.size;
    int64_t s = 1;
    for (int i = 0; i < b.rank; i++) s *= (b.shape[i] == 0 ? n : b.shape[i]);
    return s;
}

int run_impl(ah_device *d, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
             int64_t symval, bool symbolic, ah_output **outputs, int32_t *n_outputs) {
    if (!d || (!items && n_items) || !outputs || !n_outputs) return set_error(AH_ERR_INVALID, "ah_run: null argument");
    *outputs = nullptr;
    *n_outputs = 0;
    if (n_items == 0) return AH_OK;
    RunState st;
    st.dev = d;
    std::set<uint32_t> written, read_any;
    for (int i = 0; i < n_items; i++) {
        if (items[i].n_bufs < 1 || !items[i].bufs || !items[i].source)
            return set_error(AH_ERR_INVALID, "ah_run: kernel %d has no buffers or source", i);
        written.insert(items[i].bufs[0].uop_idx);
        for (int j = 1; j < items[i].n_bufs; j++) read_any.insert(items[i].bufs[j].uop_idx);
        for (int j = 0; j < items[i].n_bufs; j++) {
            const ah_buffer_desc &b = items[i].bufs[j];
            st.dtype[b.uop_idx] = b.dtype;
            st.elems[b.uop_idx] = bound_size(b, symval);
        }
    }
    // Phase A: slots sized for their largest user (4 bytes per element, executor.go:83-112).
    std::map<int, int64_t> slot_max;
    for (int i = 0; i < n_items; i++) {
        const ah_buffer_desc &o = items[i].bufs[0];
        if (o.slot >= 0) slot_max[o.slot] = std::max(slot_max[o.slot], bound_size(o, symval));
    }
    std::map<int, void *> slot_ptr;
    for (auto &kv : slot_max) {
        void *p = nullptr;
        AH_HIP(hipMalloc(&p, (size_t)std::max<int64_t>(kv.second, 1) * 4));
        st.owned.push_back(p);
        slot_ptr[kv.first] = p;
    }
    // Phase B/C: dedicated outputs and leaves.
    for (int i = 0; i < n_items; i++) {
        for (int j = 0; j < items[i].n_bufs; j++) {
            const ah_buffer_desc &b = items[i].bufs[j];
            if (st.ptr.count(b.uop_idx)) continue;
            if (j == 0 && b.slot >= 0) { st.ptr[b.uop_idx] = slot_ptr[b.slot]; continue; }
            if (j > 0 && written.count(b.uop_idx)) continue;   // produced by another item; bound when it runs
            void *p = nullptr;
            AH_HIP(hipMalloc(&p, (size_t)std::max<int64_t>(st.elems[b.uop_idx], 1) * dtype_bytes(b.dtype)));
            st.owned.push_back(p);
            st.ptr[b.uop_idx] = p;
        }
    }
    for (int i = 0; i < n_items; i++) {
        const ah_buffer_desc &o = items[i].bufs[0];
        if (!st.ptr.count(o.uop_idx)) return set_error(AH_ERR_INVALID, "ah_run: output %u unallocated", o.uop_idx);
    }
    // Upload leaves (inputs for unknown buffers are ignored, executor.go:163-165).
    for (int i = 0; i < n_inputs; i++) {
        auto it = st.ptr.find(inputs[i].uop_idx);
        if (it == st.ptr.end()) continue;
        int64_t n = std::min<int64_t>(inputs[i].n, st.elems[inputs[i].uop_idx]);
        int rc = ah_upload(d, it->second, inputs[i].data, n, st.dtype[inputs[i].uop_idx]);
        if (rc) return rc;
    }
    // Dispatch in schedule order.
    for (int i = 0; i < n_items; i++) {
        const ah_exec_item &it = items[i];
        ah_kernel *k = nullptr;
        int rc = ah_module_get(d, it.source, "kernel", &k);
        if (rc) return set_error(rc, "ah_run: kernel %d: %s", i, ah_last_error());
        std::vector<void *> ptrs;
        for (int j = 0; j < it.n_bufs; j++) {
            auto p = st.ptr.find(it.bufs[j].uop_idx);
            if (p == st.ptr.end()) return set_error(AH_ERR_INVALID, "ah_run: kernel %d: missing GPU buffer %u", i, it.bufs[j].uop_idx);
            ptrs.push_back(p->second);
        }
        std::vector<int32_t> sc;
        if (symbolic && it.n_sym_vars > 0) sc.assign(4, (int32_t)symval);   // params_n: 16-byte uniform
        uint32_t grid[3], block[3];
        for (int a = 0; a < 3; a++) {
            grid[a] = (uint32_t)std::max(1, it.workgroup_count[a]);
            block[a] = (uint32_t)std::max(1, it.local_size[a]);
        }
        if (symbolic && it.n_sym_vars > 0) {   // 1-D dispatch over the bound output (executor.go:874-898)
            int64_t out_elems = bound_size(it.bufs[0], symval);
            grid[0] = (uint32_t)((out_elems + block[0] - 1) / block[0]);
        }
        rc = ah_launch(d, k, grid, block, ptrs.data(), (int32_t)ptrs.size(), sc.data(), (int32_t)sc.size());
        if (rc) return set_error(rc, "ah_run: kernel %d: %s", i, ah_last_error());
    }
    // Read back final outputs.
    std::vector<ah_output> outs;
    for (int i = 0; i < n_items; i++) {
        const ah_buffer_desc &o = items[i].bufs[0];
        if (read_any.count(o.uop_idx)) continue;
        bool dup = false;
        for (auto &x : outs) dup |= x.uop_idx == o.uop_idx;
        if (dup) continue;
        ah_output r;
        r.uop_idx = o.uop_idx;
        r.n = st.elems[o.uop_idx];
        r.data = (float *)malloc((size_t)std::max<int64_t>(r.n, 1) * 4);
        int rc = ah_download(d, r.data, st.ptr[o.uop_idx], r.n, o.dtype);
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

}  // namespace
}  // namespace ah

using namespace ah;

extern "C" {

int ah_run(ah_device *d, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
           ah_output **outputs, int32_t *n_outputs) {
    return run_impl(d, items, n_items, inputs, n_inputs, 0, false, outputs, n_outputs);
}

int ah_run_symbolic(ah_device *d, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
                    const char *const *bind_names, const int64_t *bind_values, int32_t n_bind, ah_output **outputs,
                    int32_t *n_outputs) {
    // Like the reference, only the binding of the first symbolic item's SymVars[0] is used
    // (backend/webgpu/executor.go:817-822).
    int64_t n = -1;
    for (int i = 0; i < n_items && n < 0; i++) {
        if (items[i].n_sym_vars < 1 || !items[i].sym_vars) continue;
        for (int b = 0; b < n_bind; b++)
            if (bind_names && bind_names[b] && strcmp(bind_names[b], items[i].sym_vars[0]) == 0) n = bind_values[b];
        if (n < 0) return set_error(AH_ERR_INVALID, "ah_run_symbolic: no binding for %s", items[i].sym_vars[0]);
    }
    if (n < 0) n = 0;
    return run_impl(d, items, n_items, inputs, n_inputs, n, true, outputs, n_outputs);
}

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
    std::vector<void *> ptrs;
    auto release = [&]() { for (void *p : ptrs) hipFree(p); };
    for (int j = 0; j < item->n_bufs; j++) {
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, (size_t)std::max<int64_t>(item->bufs[j].size, 1) * dtype_bytes(item->bufs[j].dtype));
        if (e != hipSuccess) { release(); return fail_hip(e, "benchmark: hipMalloc"); }
        hipMemsetAsync(p, 0, (size_t)std::max<int64_t>(item->bufs[j].size, 1) * dtype_bytes(item->bufs[j].dtype), d->stream);
        ptrs.push_back(p);
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
