// plans.cpp — device-resident training steps for the five BASELINE configs, plus the direct kernel
// entry points of the C ABI.
//
// The reference's step is: build the graph, tensor.Backward, then one tensor.Realize per gradient
// (each re-running the forward kernels that gradient needs) and a host-side SGD over f32 masters
// (examples/mlp.go:112-142, tensor/nn/nn.go:56-106). Here one step enqueues a fixed kernel list on the
// device stream: the forward once, every gradient once, and SGD fused into the weight-gradient GEMM
// epilogues, with parameters resident in HBM across steps.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>
#include <vector>

#include "ah_internal.h"
#include "conv.h"
#include "convnet.h"
#include "mlpce.h"
#include "gemm.h"
#include "itemops.h"
#include "rowops.h"

using namespace ah;

// Steps per hipGraph in ah_trainer_steps (the rest of n runs as one shorter graph).
constexpr int kMaxGraphSteps = 16;

struct ah_trainer {
    ah_device *dev = nullptr;
    int kind = 0;
    std::vector<int64_t> dims;
    float lr = 0.0f;
    std::vector<void *> allocs;
    int probe_index = -1;   // first launch a probe brackets (-1: no probe)
    int probe_last = -1;    // last launch it brackets; probe_index - 1 brackets nothing (event cost alone)
    int launch_idx = 0;
    std::vector<hipEvent_t> ev_a, ev_b;
    size_t n_probe = 0;
    std::map<int64_t, ah_graph *> graphs;
    bool record_names = false;
    std::vector<std::string> names;   // launch names of the last ah_trainer_kernel_count

    virtual ~ah_trainer() {
        if (dev) hipStreamSynchronize(dev->stream);
        for (auto &kv : graphs) ah_graph_destroy(kv.second);
        for (void *p : allocs) hipFree(p);
        for (auto e : ev_a) hipEventDestroy(e);
        for (auto e : ev_b) hipEventDestroy(e);
    }
    virtual int set(int slot, const void *host, int64_t n) = 0;
    virtual int get(int slot, void *host, int64_t n) = 0;
    virtual int enqueue(int64_t batch, int flags) = 0;
    // Work before a batch's first step, outside any capture (tuning); called before every step.
    virtual int prepare(int64_t) { return AH_OK; }
    virtual int max_batch() const { return (int)dims[0]; }

    template <class T>
    int alloc(T **p, size_t n) {
        void *q = nullptr;
        hipError_t e = hipMalloc(&q, std::max<size_t>(n, 1) * sizeof(T));
        if (e != hipSuccess) return fail_hip(e, "hipMalloc (trainer buffer)");
        allocs.push_back(q);
        *p = (T *)q;
        return AH_OK;
    }

    // Every kernel of a step goes through here so a probe can bracket launches probe_index..probe_last.
    template <class F>
    int launch(const char *what, F &&f) {
        const bool open = probe_index >= 0 && launch_idx == probe_index;
        if (open) {
            if (n_probe >= ev_a.size()) {
                hipEvent_t a, b;
                // timing-only events: no system-scope fence (cache writeback and invalidate) at
                // record time, which would add to the bracketed kernels' measured duration
                AH_HIP(hipEventCreateWithFlags(&a, hipEventDisableSystemFence));
                AH_HIP(hipEventCreateWithFlags(&b, hipEventDisableSystemFence));
                ev_a.push_back(a);
                ev_b.push_back(b);
            }
            AH_HIP(hipEventRecord(ev_a[n_probe], dev->stream));
            if (probe_last < probe_index) {
                AH_HIP(hipEventRecord(ev_b[n_probe], dev->stream));
                n_probe++;
            }
        }
        if (record_names) names.push_back(what);
        hipError_t e = f();
        if (e != hipSuccess) return set_error(AH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
        if (probe_index >= 0 && probe_last >= probe_index && launch_idx == probe_last) {
            AH_HIP(hipEventRecord(ev_b[n_probe], dev->stream));
            n_probe++;
        }
        launch_idx++;
        return AH_OK;
    }
};

#define LAUNCH(name, expr)                                    \
    do {                                                      \
        int rc_ = launch(name, [&]() -> hipError_t { return (expr); }); \
        if (rc_ != AH_OK) return rc_;                         \
    } while (0)

static int copy_in(ah_device *d, void *dst, const void *src, size_t bytes) {
    AH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, d->stream));
    AH_HIP(hipStreamSynchronize(d->stream));
    return AH_OK;
}
static int copy_out(ah_device *d, void *dst, const void *src, size_t bytes) {
    AH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, d->stream));
    AH_HIP(hipStreamSynchronize(d->stream));
    return AH_OK;
}
// f32 host array -> f16 device array with the reference codec (uop/dtype.go:392).
static int copy_in_f16(ah_device *d, half_t *dst, const float *src, size_t n) {
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; i++) h[i] = ah_f32_to_f16(src[i]);
    return copy_in(d, dst, h.data(), n * 2);
}

// ── GEMM variant tuning ─────────────────────────────────────────────────────

static std::string tune_key(const GemmDesc &g) {
    char b[96];
    snprintf(b, sizeof b, "%d/%d/%d/%d/%d/%d%s", g.dtype, g.ta, g.tb, g.M, g.N, g.K, g.A2 ? "/2" : "");
    return b;
}

// Configurations of the f32 tiled kernel the tuner times: (tile, k-groups, splits), 0 meaning the
// shape's automatic choice of that parameter; entry 0 leaves all three to the shape. A fixed k-group
// count with splits 0 runs without a split of K across workgroups.
struct F32Cfg {
    int tile, kg, splits;
};
static const std::vector<F32Cfg> &f32_cfgs() {
    static const std::vector<F32Cfg> v = [] {
        std::vector<F32Cfg> c{{0, 0, 0}};
        for (int tile : {64, 128})
            for (int kg : {0, 1, 2, 4}) {
                if (kg && !gemm32_kgroups_ok(tile, kg)) continue;
                for (int sp : {0, 1, 2, 4, 8, 16}) {
                    if (kg && sp == 0) continue;   // the same launch as splits 1
                    c.push_back({tile, kg, sp});
                }
            }
        for (int i = 0; i < kGemm32dConfigs; i++) c.push_back({kGemm32dBase + i, 0, 0});   // direct-to-LDS stages
        for (int i = 0; i < kGemm32dConfigs; i++)                                           // ... splitting K
            for (int sp : {2, 4, 8}) c.push_back({kGemm32dBase + i, 0, sp});
        return c;
    }();
    return v;
}

// Launch with the tuned variant (f16) or configuration (f32) when the caller left the choice open, and
// with the device's split-K workspace (used by the f32 tiled kernel for shapes with few tiles and a
// long K).
static hipError_t gemm_run(ah_device *dev, GemmDesc g, hipStream_t s) {
    if (g.variant == 0 && g.dtype == GEMM_F16) {
        auto it = dev->gemm_variant.find(tune_key(g));
        if (it != dev->gemm_variant.end()) g.variant = it->second;
    }
    if (g.dtype == GEMM_F32 && g.tile == 0 && g.kgroups == 0 && g.splits == 0) {
        auto it = dev->gemm_variant.find(tune_key(g));
        if (it != dev->gemm_variant.end() && it->second > 0 && it->second < (int)f32_cfgs().size()) {
            const F32Cfg &c = f32_cfgs()[it->second];
            g.tile = c.tile; g.kgroups = c.kg; g.splits = c.splits;
        }
    }
    if (dev->splitk_ws) {
        const size_t sync_bytes = (size_t)kSplitKMaxTiles * 2 * sizeof(int);
        g.sk_sync = (int *)dev->splitk_ws;
        g.sk_part = (float *)((char *)dev->splitk_ws + sync_bytes);
        g.sk_cap = kSplitKPartFloats;
    }
    return gemm_launch(g, s);
}

hipError_t ah::gemm_dispatch(ah_device *dev, const GemmDesc &g) { return gemm_run(dev, g, dev->stream); }

// Times every f16 variant of g (as given: its epilogue runs on whatever outputs g names) and caches
// the fastest for g's shape. Two passes over the variants, each variant's time the lower of its two
// means of `iters` launches, so one disturbed measurement does not decide the choice.
static int tune_gemm_f32(ah_device *dev, GemmDesc g, int iters, int *best, double *best_us, bool same_bits);
static int tune_gemm(ah_device *dev, GemmDesc g, int iters, int *best, double *best_us) {
    if (g.dtype == GEMM_F32) return tune_gemm_f32(dev, g, iters, best, best_us, false);
    if (g.dtype != GEMM_F16) return set_error(AH_ERR_UNSUPPORTED, "gemm tuning covers the f16 and f32 kernels");
    if (iters <= 0) return set_error(AH_ERR_INVALID, "gemm tuning: iterations must be > 0");
    hipEvent_t e0, e1;
    AH_HIP(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence));   // timing only
    AH_HIP(hipEventCreateWithFlags(&e1, hipEventDisableSystemFence));
    std::vector<float> t(kGemm16Variants + 1, 0.0f);
    hipError_t err = hipSuccess;
    for (int pass = 0; pass < 2 && err == hipSuccess; pass++) {
        for (int v = 1; v <= kGemm16Variants && err == hipSuccess; v++) {
            g.variant = v;
            err = gemm_launch(g, dev->stream);
            if (err == hipSuccess) err = hipEventRecord(e0, dev->stream);
            for (int i = 0; i < iters && err == hipSuccess; i++) err = gemm_launch(g, dev->stream);
            if (err == hipSuccess) err = hipEventRecord(e1, dev->stream);
            if (err == hipSuccess) err = hipEventSynchronize(e1);
            float ms = 0.0f;
            if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
            if (err == hipSuccess && (pass == 0 || ms < t[v])) t[v] = ms;
        }
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (err != hipSuccess) return fail_hip(err, "gemm tuning");
    int bv = 1;
    for (int v = 2; v <= kGemm16Variants; v++)
        if (t[v] < t[bv]) bv = v;
    dev->gemm_variant[tune_key(g)] = bv;
    if (best) *best = bv;
    if (best_us) *best_us = t[bv] * 1000.0 / iters;
    return AH_OK;
}

// The f32 counterpart: times every configuration of f32_cfgs() the same way (two passes, the lower of
// each configuration's two means) and caches the fastest one's index for g's shape (0: the automatic
// choice). Configurations add K in different orders, so results differ at the rounding level. With
// same_bits, a configuration is a candidate only when its output is bit-identical to the automatic
// choice's (BEAM's value guard, codegen/beam.go:410-451), checked on hash-filled operands of g's shape
// and layout: the choice then changes only the speed, never the result, whichever configuration a
// noisy timing picks.
static int tune_gemm_f32(ah_device *dev, GemmDesc g, int iters, int *best, double *best_us, bool same_bits) {
    if (iters <= 0) return set_error(AH_ERR_INVALID, "gemm tuning: iterations must be > 0");
    const std::vector<F32Cfg> &cfgs = f32_cfgs();
    if (dev->splitk_ws) {
        const size_t sync_bytes = (size_t)kSplitKMaxTiles * 2 * sizeof(int);
        g.sk_sync = (int *)dev->splitk_ws;
        g.sk_part = (float *)((char *)dev->splitk_ws + sync_bytes);
        g.sk_cap = kSplitKPartFloats;
    }
    std::vector<char> admitted(cfgs.size(), 1);
    if (same_bits) {
        // the guard runs on hash-filled copies of g's operands (real operands may still be all zero),
        // writing into scratch: C, or the gradient output of an SGD epilogue
        GemmDesc q = g;
        const long na = (long)(g.ta ? g.K : g.M) * g.lda, nb = (long)(g.tb ? g.K : g.N) * g.ldb;
        const long nc = (long)(g.M - 1) * g.ldc + g.N, nx = g.aux ? (long)(g.M - 1) * g.ldaux + g.N : 0;
        const long total = na + nb + 3 * nc + nx + (g.bias ? g.N : 0) + 64;
        float *scr = nullptr;
        int *flag = nullptr;
        hipError_t e = hipMalloc(&scr, (size_t)total * 4);
        if (e == hipSuccess) e = hipMalloc((void **)&flag, sizeof(int));
        if (e == hipSuccess) e = fill_hash(scr, nullptr, total, 11u, 1.0f, dev->stream);
        float *p = scr;
        q.A = p; p += na;
        q.B = p; p += nb;
        float *out = p, *ref = p + nc, *w32 = p + 2 * nc;
        p += 3 * nc;
        if (g.aux) { q.aux = p; p += nx; }
        if (g.bias) q.bias = p;
        q.colsum = nullptr;
        q.lossacc = nullptr;
        if (g.epi == EPI_SGD) { q.W32 = w32; q.gout = out; q.C = nullptr; q.W16 = nullptr; }
        else q.C = out;
        q.tile = q.kgroups = q.splits = 0;
        if (e == hipSuccess) e = gemm_launch(q, dev->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(ref, out, (size_t)nc * 4, hipMemcpyDeviceToDevice, dev->stream);
        for (size_t v = 1; v < cfgs.size() && e == hipSuccess; v++) {
            q.tile = cfgs[v].tile; q.kgroups = cfgs[v].kg; q.splits = cfgs[v].splits;
            e = gemm_launch(q, dev->stream);
            if (e == hipSuccess) e = words_differ(out, ref, nc, flag, dev->stream);
            int differs = 1;
            if (e == hipSuccess) e = hipMemcpyAsync(&differs, flag, sizeof(int), hipMemcpyDeviceToHost, dev->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
            admitted[v] = e == hipSuccess && differs == 0;
        }
        if (scr) hipFree(scr);
        if (flag) hipFree(flag);
        if (e != hipSuccess) return fail_hip(e, "gemm tuning (f32 bit-identity guard)");
    }
    hipEvent_t e0, e1;
    AH_HIP(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence));   // timing only
    AH_HIP(hipEventCreateWithFlags(&e1, hipEventDisableSystemFence));
    std::vector<float> t(cfgs.size(), 0.0f);
    hipError_t err = hipSuccess;
    for (int pass = 0; pass < 2 && err == hipSuccess; pass++) {
        for (size_t v = 0; v < cfgs.size() && err == hipSuccess; v++) {
            if (!admitted[v]) { t[v] = 1e30f; continue; }
            g.tile = cfgs[v].tile; g.kgroups = cfgs[v].kg; g.splits = cfgs[v].splits;
            err = gemm_launch(g, dev->stream);
            if (err == hipSuccess) err = hipEventRecord(e0, dev->stream);
            for (int i = 0; i < iters && err == hipSuccess; i++) err = gemm_launch(g, dev->stream);
            if (err == hipSuccess) err = hipEventRecord(e1, dev->stream);
            if (err == hipSuccess) err = hipEventSynchronize(e1);
            float ms = 0.0f;
            if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
            if (err == hipSuccess && (pass == 0 || ms < t[v])) t[v] = ms;
        }
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (err != hipSuccess) return fail_hip(err, "gemm tuning (f32)");
    int bv = 0;
    for (size_t v = 1; v < cfgs.size(); v++)
        if (t[v] < t[bv]) bv = (int)v;
    g.tile = g.kgroups = g.splits = 0;
    dev->gemm_variant[tune_key(g)] = bv;
    if (best) *best = bv;
    if (best_us) *best_us = t[bv] * 1000.0 / iters;
    return AH_OK;
}

static GemmDesc gdesc(int dtype, int epi, int ta, int tb, int M, int N, int K, const void *A, long lda,
                      const void *B, long ldb, void *C, long ldc) {
    GemmDesc g;
    memset(&g, 0, sizeof g);
    g.dtype = dtype; g.epi = epi; g.ta = ta; g.tb = tb; g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc; g.scale = 1.0f;
    return g;
}

// ── configs 1 and 4: Linear(D->H) ReLU Linear(H->C), softmax-CE ─────────────

struct MlpCeTrainer : ah_trainer {
    int Bmax, D, H, C;
    float *x, *W1, *b1, *W2, *b2, *H1, *Z2, *dZ2, *dZ1, *rowloss, *acc, *loss, *gW1, *gb1, *gW2, *gb2;
    float *dbpart = nullptr;   // softmax_ce_cols' partial rows of the output bias gradient (C <= kSoftmaxColsMaxC)
    // dH1's column sums (the hidden bias gradient) as one partial row per 32-row block a wave of the
    // masked contraction starts (GemmDesc::colsum_ld): plain stores summed by the tail in row order and
    // re-zeroed there, so db1 does not depend on the order in which workgroups finish
    float *db1part = nullptr;
    int32_t *lab;
    bool fused = false;   // the three-kernel step of mlpce.h
    int init() {
        Bmax = (int)dims[0]; D = (int)dims[1]; H = (int)dims[2]; C = (int)dims[3];
        if (Bmax <= 0 || D <= 0 || H <= 0 || C <= 0) return set_error(AH_ERR_INVALID, "MLP_CE: bad dims");
        int rc = AH_OK;
        rc |= alloc(&x, (size_t)Bmax * D); rc |= alloc(&lab, Bmax);
        rc |= alloc(&W1, (size_t)H * D); rc |= alloc(&b1, H); rc |= alloc(&W2, (size_t)C * H); rc |= alloc(&b2, C);
        rc |= alloc(&H1, (size_t)Bmax * H); rc |= alloc(&Z2, (size_t)Bmax * C); rc |= alloc(&dZ2, (size_t)Bmax * C);
        rc |= alloc(&dZ1, (size_t)Bmax * H); rc |= alloc(&rowloss, Bmax); rc |= alloc(&acc, H + C);
        rc |= alloc(&loss, 1); rc |= alloc(&gW1, (size_t)H * D); rc |= alloc(&gb1, H);
        rc |= alloc(&gW2, (size_t)C * H); rc |= alloc(&gb2, C);
        if (C <= kSoftmaxColsMaxC) rc |= alloc(&dbpart, (size_t)softmax_ce_cols_blocks(Bmax) * C);
        rc |= alloc(&db1part, (size_t)((Bmax + 31) / 32) * H);
        fused = mlpce_fused_ok(Bmax, D, H, C);
        if (rc) return AH_ERR_HIP;
        AH_HIP(hipMemset(acc, 0, sizeof(float) * (H + C)));
        AH_HIP(hipMemset(db1part, 0, sizeof(float) * ((Bmax + 31) / 32) * H));
        return AH_OK;
    }
    int set(int slot, const void *h, int64_t n) override {
        struct { void *p; int64_t n; } t[] = {{x, (int64_t)Bmax * D}, {lab, Bmax}, {W1, (int64_t)H * D}, {b1, H},
                                              {W2, (int64_t)C * H}, {b2, C}};
        if (slot < 0 || slot > 5) return set_error(AH_ERR_INVALID, "MLP_CE: slot %d not settable", slot);
        if (n > t[slot].n) return set_error(AH_ERR_INVALID, "MLP_CE: slot %d: %lld > %lld", slot, (long long)n, (long long)t[slot].n);
        return copy_in(dev, t[slot].p, h, (size_t)n * 4);
    }
    int get(int slot, void *h, int64_t n) override {
        struct { void *p; int64_t n; } t[] = {{x, (int64_t)Bmax * D}, {lab, Bmax}, {W1, (int64_t)H * D}, {b1, H},
                                              {W2, (int64_t)C * H}, {b2, C}, {loss, 1}, {gW1, (int64_t)H * D},
                                              {gb1, H}, {gW2, (int64_t)C * H}, {gb2, C}, {H1, (int64_t)Bmax * H}};
        if (slot < 0 || slot > 11) return set_error(AH_ERR_INVALID, "MLP_CE: bad slot %d", slot);
        if (n > t[slot].n) return set_error(AH_ERR_INVALID, "MLP_CE: slot %d too small", slot);
        return copy_out(dev, h, t[slot].p, (size_t)n * 4);
    }
    // Before a batch's first GEMM-based step outside a capture: tune each f32 contraction's (tile,
    // k-groups, splits) for shapes the device has not tuned. Each runs with its own epilogue into
    // buffers the step rewrites (the weight updates into the gradient outputs, with lr 0); the
    // bias-gradient accumulator it touches is re-zeroed.
    std::set<int> tuned;
    int prepare(int64_t batch) override {
        const int B = (int)batch;
        if (fused || mlp_small_ok(B, D, H, C) || tuned.count(B)) return AH_OK;
        const char *off = getenv("AH_GEMM_TUNE");   // "0": keep the automatic choices
        if (off && *off == '0') return AH_OK;
        // a caller capturing the device stream gets the automatic choices (timing would end its capture)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        AH_HIP(hipStreamIsCapturing(dev->stream, &cs));
        if (cs != hipStreamCaptureStatusNone) return AH_OK;
        GemmDesc g[5] = {gdesc(GEMM_F32, EPI_BIAS_RELU, 0, 0, B, H, D, x, D, W1, D, H1, H),
                         gdesc(GEMM_F32, EPI_BIAS, 0, 0, B, C, H, H1, H, W2, H, Z2, C),
                         gdesc(GEMM_F32, EPI_MASK, 0, 1, B, H, C, dZ2, C, W2, H, dZ1, H),
                         gdesc(GEMM_F32, EPI_SGD, 1, 1, C, H, B, dZ2, C, H1, H, nullptr, H),
                         gdesc(GEMM_F32, EPI_SGD, 1, 1, H, D, B, dZ1, H, x, D, nullptr, D)};
        g[0].bias = b1;
        g[1].bias = b2;
        g[2].aux = H1; g[2].ldaux = H; g[2].colsum = db1part; g[2].colsum_ld = H;
        g[3].W32 = gW2; g[3].lr = 0.0f;
        g[4].W32 = gW1; g[4].lr = 0.0f;
        // Only configurations that add K in the automatic choice's order are candidates, so the step's
        // results do not depend on which of them timing noise selects (AH_GEMM_TUNE_ANY_ORDER=1 admits
        // every configuration: faster on some shapes, results then equal only to rounding).
        const char *any = getenv("AH_GEMM_TUNE_ANY_ORDER");
        const bool same_bits = !(any && *any == '1');
        int rc = AH_OK;
        for (GemmDesc &d : g)
            if (rc == AH_OK && !dev->gemm_variant.count(tune_key(d))) rc = tune_gemm_f32(dev, d, 3, nullptr, nullptr, same_bits);
        if (rc) return rc;
        AH_HIP(hipMemsetAsync(acc, 0, sizeof(float) * (H + C), dev->stream));
        AH_HIP(hipMemsetAsync(db1part, 0, sizeof(float) * ((Bmax + 31) / 32) * H, dev->stream));
        tuned.insert(B);
        return AH_OK;
    }
    int enqueue(int64_t batch, int flags) override {
        const int B = (int)batch;
        hipStream_t s = dev->stream;
        const bool sg = flags & AH_STEP_STORE_GRADS;
        const float a = (float)(-1.0 / (double)B);
        if (fused) {
            MlpSgd u{W1, b1, W2, b2, sg ? gW1 : nullptr, sg ? gb1 : nullptr, sg ? gW2 : nullptr, sg ? gb2 : nullptr,
                     lr, a, loss};
            LAUNCH("hidden", mlpce_hidden(x, W1, b1, B, D, H, H1, s));
            LAUNCH("head", mlpce_head(lab, H1, W2, b2, B, H, C, a, dZ2, dZ1, rowloss, s));
            LAUNCH("grad", mlpce_grad(x, H1, dZ2, dZ1, rowloss, B, D, H, C, u, s));
            return AH_OK;
        }
        if (mlp_small_ok(B, D, H, C)) {
            MlpSgd u{W1, b1, W2, b2, sg ? gW1 : nullptr, sg ? gb1 : nullptr, sg ? gW2 : nullptr, sg ? gb2 : nullptr,
                     lr, a, loss};
            LAUNCH("fc1", mlp_small_step(x, lab, B, D, H, C, a, H1, Z2, dZ2, dZ1, rowloss, u, s, 0));
            LAUNCH("fc2", mlp_small_step(x, lab, B, D, H, C, a, H1, Z2, dZ2, dZ1, rowloss, u, s, 1));
            LAUNCH("dH1", mlp_small_step(x, lab, B, D, H, C, a, H1, Z2, dZ2, dZ1, rowloss, u, s, 2));
            LAUNCH("grad", mlp_small_step(x, lab, B, D, H, C, a, H1, Z2, dZ2, dZ1, rowloss, u, s, 3));
            return AH_OK;
        }
        float *db2 = acc + H;
        GemmDesc g1 = gdesc(GEMM_F32, EPI_BIAS_RELU, 0, 0, B, H, D, x, D, W1, D, H1, H);
        g1.bias = b1;
        LAUNCH("fc1", gemm_run(dev, g1, s));
        GemmDesc g2 = gdesc(GEMM_F32, EPI_BIAS, 0, 0, B, C, H, H1, H, W2, H, Z2, C);
        g2.bias = b2;
        LAUNCH("fc2", gemm_run(dev, g2, s));
        if (dbpart) {
            LAUNCH("softmax_ce", softmax_ce_cols(Z2, lab, B, C, a, dZ2, rowloss, dbpart, s));
        } else {
            LAUNCH("softmax_ce", softmax_ce(Z2, lab, B, C, a, dZ2, rowloss, s));
            LAUNCH("db2", colsum_add(dZ2, B, C, C, db2, s));
        }
        GemmDesc g3 = gdesc(GEMM_F32, EPI_MASK, 0, 1, B, H, C, dZ2, C, W2, H, dZ1, H);
        g3.aux = H1; g3.ldaux = H; g3.colsum = db1part; g3.colsum_ld = H;
        LAUNCH("dH1", gemm_run(dev, g3, s));
        GemmDesc g4 = gdesc(GEMM_F32, EPI_SGD, 1, 1, C, H, B, dZ2, C, H1, H, nullptr, H);
        g4.W32 = W2; g4.lr = lr; g4.gout = sg ? gW2 : nullptr;
        GemmDesc g5 = gdesc(GEMM_F32, EPI_SGD, 1, 1, H, D, B, dZ1, H, x, D, nullptr, D);
        g5.W32 = W1; g5.lr = lr; g5.gout = sg ? gW1 : nullptr;
        LAUNCH("dW1", gemm_run(dev, g5, s));
        LAUNCH("dW2", gemm_run(dev, g4, s));
        TailArgs ta{};
        ta.seg[0] = {b2, nullptr, db2, sg ? gb2 : nullptr, C, 1.0f};
        if (dbpart) {   // the bias gradient as softmax_ce_cols' partial rows, rewritten every step
            ta.seg[0].acc = dbpart;
            ta.seg[0].acc_rows = softmax_ce_cols_blocks(B);
            ta.seg[0].acc_ld = C;
            ta.seg[0].keep = 1;
        }
        ta.seg[1] = {b1, nullptr, db1part, sg ? gb1 : nullptr, H, 1.0f, (B + 31) / 32, (long)H, 0};
        ta.nseg = 2; ta.lr = lr; ta.loss_mode = 2; ta.loss_scale = a; ta.rowloss = rowloss; ta.nrow = B; ta.loss_out = loss;
        LAUNCH("tail", step_tail(ta, s));
        return AH_OK;
    }
};

// ── config 3: f16 three-layer MLP with MSE ──────────────────────────────────
// The loss adjoint 2*d/(B*D3) is carried as d (exact f16) through the backward GEMMs and the factor
// 2/(B*D3) is applied in the f32 weight-update epilogues; this keeps f16 MFMA operands in range
// (the raw adjoint, ~1e-7 at B*D3 = 2^22, is below f16's normal range).

// The unpaired config-3 step's launch order (contraction indices 0-7: fc1, fc2, fc3, dH2, dW3, dH1, dW2,
// dW1): the backward runs dH2, dH1, dW1, dW3, dW2, so dH1 reads dH2's output and dW1 dH1's while the
// Infinity Cache still holds them. kMlp3LaunchPos[i] is contraction i's position.
constexpr int kMlp3Order[8] = {0, 1, 2, 3, 5, 7, 4, 6};
constexpr int mlp3_launch_pos(int i) {
    int p = 0;
    while (kMlp3Order[p] != i) p++;
    return p;
}
constexpr int kMlp3LaunchPos[8] = {mlp3_launch_pos(0), mlp3_launch_pos(1), mlp3_launch_pos(2), mlp3_launch_pos(3),
                                   mlp3_launch_pos(4), mlp3_launch_pos(5), mlp3_launch_pos(6), mlp3_launch_pos(7)};

struct Mlp3Trainer : ah_trainer {
    int B, D0, D1, D2, D3;
    half_t *X, *T, *W1h, *W2h, *W3h, *b1h, *b2h, *b3h, *H1, *H2, *Dd, *dZ2, *dZ1;
    // f32-adjoint mode (dims[5] = 1): the masked adjoints dZ2 and dZ1 are kept as two f16 planes,
    // hi = f16(v) in dZ2/dZ1 and lo = f16(v - hi) here, and the contractions that read them (dH1, dW2,
    // dW1) run over both planes (GemmDesc::A2). The products are then the reference's f32-adjoint ones
    // (tensor/ops.go:74-79, tensor/gradient_ruleset.go:114-122) to about 22 bits of the adjoint.
    bool exact = false;
    half_t *dZ2lo = nullptr, *dZ1lo = nullptr;
    float *W1, *W2, *W3, *b1, *b2, *b3, *acc, *loss, *lsum, *gW1, *gW2, *gW3, *gb1, *gb2, *gb3;
    // Paired launches (gemm16_pair.hip): pair 0 runs dW3 split over K beside dH1, pair 1 dW1 split
    // over K beside dW2. pair_v[p] is the variant of pair p (0: the two contractions launch apart),
    // chosen by timing whole steps at creation.
    static constexpr int kPairSplit = 4;
    int pair_v[2] = {0, 0};
    int *pair_count = nullptr;   // split-K arrival counters (zero between launches)
    float *pair_part = nullptr;  // split-K partial tiles
    long pair_part_floats = 0;
    int init() {
        B = (int)dims[0]; D0 = (int)dims[1]; D1 = (int)dims[2]; D2 = (int)dims[3]; D3 = (int)dims[4];
        if (B <= 0 || D0 <= 0 || D1 <= 0 || D2 <= 0 || D3 <= 0) return set_error(AH_ERR_INVALID, "MLP3: bad dims");
        if (dims.size() > 5 && dims[5] != 0 && dims[5] != 1) return set_error(AH_ERR_INVALID, "MLP3: dims[5] (adjoint precision) is 0 or 1");
        exact = dims.size() > 5 && dims[5] == 1;
        int rc = 0;
        if (exact) { rc |= alloc(&dZ2lo, (size_t)B * D2); rc |= alloc(&dZ1lo, (size_t)B * D1); }
        rc |= alloc(&X, (size_t)B * D0); rc |= alloc(&T, (size_t)B * D3);
        rc |= alloc(&W1, (size_t)D1 * D0); rc |= alloc(&W1h, (size_t)D1 * D0);
        rc |= alloc(&W2, (size_t)D2 * D1); rc |= alloc(&W2h, (size_t)D2 * D1);
        rc |= alloc(&W3, (size_t)D3 * D2); rc |= alloc(&W3h, (size_t)D3 * D2);
        rc |= alloc(&b1, D1); rc |= alloc(&b1h, D1); rc |= alloc(&b2, D2); rc |= alloc(&b2h, D2);
        rc |= alloc(&b3, D3); rc |= alloc(&b3h, D3);
        rc |= alloc(&H1, (size_t)B * D1); rc |= alloc(&H2, (size_t)B * D2); rc |= alloc(&Dd, (size_t)B * D3);
        rc |= alloc(&dZ2, (size_t)B * D2); rc |= alloc(&dZ1, (size_t)B * D1);
        rc |= alloc(&acc, acc_floats()); rc |= alloc(&loss, 1); rc |= alloc(&lsum, 1);
        rc |= alloc(&gW1, (size_t)D1 * D0); rc |= alloc(&gW2, (size_t)D2 * D1); rc |= alloc(&gW3, (size_t)D3 * D2);
        rc |= alloc(&gb1, D1); rc |= alloc(&gb2, D2); rc |= alloc(&gb3, D3);
        // the split contractions are dW3 [D3 x D2] and dW1 [D1 x D0], in whole 256x256 tiles
        const long split_tiles = std::max((long)(D3 / 256) * (D2 / 256), (long)(D1 / 256) * (D0 / 256));
        if (split_tiles > 0) {
            pair_part_floats = split_tiles * kPairSplit * 65536;
            rc |= alloc(&pair_count, split_tiles);
            rc |= alloc(&pair_part, pair_part_floats);
        }
        if (rc) return AH_ERR_HIP;
        AH_HIP(hipMemset(acc, 0, sizeof(float) * acc_floats()));
        if (pair_count) AH_HIP(hipMemset(pair_count, 0, sizeof(int) * split_tiles));
        return tune();
    }
    // Bias-gradient and loss accumulators as deterministic per-wave partials (GemmDesc::colsum_ld,
    // loss_ld): R = ceil(B/32) row blocks of db1 [D1], db2 [D2], db3 [D3], then R x L loss partials
    // (L = ceil(D3/32)); the step tail sums them in row order and re-zeroes them.
    int rblocks() const { return (B + 31) / 32; }
    int lblocks() const { return (D3 + 31) / 32; }
    size_t acc_floats() const { return (size_t)rblocks() * (D1 + D2 + D3 + lblocks()); }
    float *db1p() const { return acc; }
    float *db2p() const { return acc + (size_t)rblocks() * D1; }
    float *db3p() const { return acc + (size_t)rblocks() * (D1 + D2); }
    float *lossp() const { return acc + (size_t)rblocks() * (D1 + D2 + D3); }
    int max_batch() const override { return B; }
    int set(int slot, const void *h, int64_t n) override {
        const float *f = (const float *)h;
        auto need = [&](int64_t want) { return n == want ? AH_OK : set_error(AH_ERR_INVALID, "MLP3: slot %d wants %lld values", slot, (long long)want); };
        int rc;
        switch (slot) {
            case 0: if ((rc = need((int64_t)B * D0))) return rc; return copy_in_f16(dev, X, f, n);
            case 1: if ((rc = need((int64_t)B * D3))) return rc; return copy_in_f16(dev, T, f, n);
            case 2: case 4: case 6: {
                float *w = slot == 2 ? W1 : slot == 4 ? W2 : W3;
                half_t *wh = slot == 2 ? W1h : slot == 4 ? W2h : W3h;
                int64_t want = slot == 2 ? (int64_t)D1 * D0 : slot == 4 ? (int64_t)D2 * D1 : (int64_t)D3 * D2;
                if ((rc = need(want))) return rc;
                if ((rc = copy_in(dev, w, f, (size_t)n * 4))) return rc;
                return copy_in_f16(dev, wh, f, n);
            }
            case 3: case 5: case 7: {
                float *b = slot == 3 ? b1 : slot == 5 ? b2 : b3;
                half_t *bh = slot == 3 ? b1h : slot == 5 ? b2h : b3h;
                int64_t want = slot == 3 ? D1 : slot == 5 ? D2 : D3;
                if ((rc = need(want))) return rc;
                if ((rc = copy_in(dev, b, f, (size_t)n * 4))) return rc;
                return copy_in_f16(dev, bh, f, n);
            }
            default: return set_error(AH_ERR_INVALID, "MLP3: slot %d not settable", slot);
        }
    }
    int get(int slot, void *h, int64_t n) override {
        struct { void *p; int64_t n; } t[] = {{nullptr, 0}, {nullptr, 0}, {W1, (int64_t)D1 * D0}, {b1, D1},
            {W2, (int64_t)D2 * D1}, {b2, D2}, {W3, (int64_t)D3 * D2}, {b3, D3}, {loss, 1},
            {gW1, (int64_t)D1 * D0}, {gb1, D1}, {gW2, (int64_t)D2 * D1}, {gb2, D2}, {gW3, (int64_t)D3 * D2}, {gb3, D3},
            {lsum, 1}};
        if (slot >= 16 && slot <= 18) {   // the step's f16 activations and loss adjoint, widened to f32
            const half_t *src = slot == 16 ? H1 : slot == 17 ? H2 : Dd;
            const int64_t cap = (int64_t)B * (slot == 16 ? D1 : slot == 17 ? D2 : D3);
            if (n > cap) return set_error(AH_ERR_INVALID, "MLP3: slot %d too small", slot);
            return ah_download(dev, (float *)h, src, n, AH_F16);
        }
        if (slot < 2 || slot > 15) return set_error(AH_ERR_INVALID, "MLP3: bad slot %d", slot);
        if (n > t[slot].n) return set_error(AH_ERR_INVALID, "MLP3: slot %d too small", slot);
        return copy_out(dev, h, t[slot].p, (size_t)n * 4);
    }
    // The step's eight contractions, in launch order (fc1 fc2 fc3_mse dH2 dW3 dH1 dW2 dW1).
    static constexpr int kGemms = 8;
    GemmDesc gemm(int i, bool sg) const {
        const float sc = (float)(1.0 / ((double)B * (double)D3));
        const float bs = 2.0f * sc;
        float *db1 = db1p(), *db2 = db2p(), *db3 = db3p(), *lacc = lossp();
        GemmDesc g;
        switch (i) {
            case 0: g = gdesc(GEMM_F16, EPI_BIAS_RELU, 0, 0, B, D1, D0, X, D0, W1h, D0, H1, D1); g.bias = b1h; break;
            case 1: g = gdesc(GEMM_F16, EPI_BIAS_RELU, 0, 0, B, D2, D1, H1, D1, W2h, D1, H2, D2); g.bias = b2h; break;
            case 2:
                g = gdesc(GEMM_F16, EPI_MSE, 0, 0, B, D3, D2, H2, D2, W3h, D2, Dd, D3);
                g.bias = b3h; g.aux = T; g.ldaux = D3; g.colsum = db3; g.lossacc = lacc;
                g.colsum_ld = D3; g.loss_ld = lblocks();
                break;
            case 3:
                g = gdesc(GEMM_F16, EPI_MASK, 0, 1, B, D2, D3, Dd, D3, W3h, D2, dZ2, D2);
                g.aux = H2; g.ldaux = D2; g.colsum = db2; g.colsum_ld = D2;
                g.C2 = dZ2lo;
                break;
            case 4:
                g = gdesc(GEMM_F16, EPI_SGD, 1, 1, D3, D2, B, Dd, D3, H2, D2, nullptr, D2);
                g.scale = bs; g.W32 = W3; g.W16 = W3h; g.lr = lr; g.gout = sg ? gW3 : nullptr;
                break;
            case 5:
                g = gdesc(GEMM_F16, EPI_MASK, 0, 1, B, D1, D2, dZ2, D2, W2h, D1, dZ1, D1);
                g.aux = H1; g.ldaux = D1; g.colsum = db1; g.colsum_ld = D1;
                g.A2 = dZ2lo; g.C2 = dZ1lo;
                break;
            case 6:
                g = gdesc(GEMM_F16, EPI_SGD, 1, 1, D2, D1, B, dZ2, D2, H1, D1, nullptr, D1);
                g.scale = bs; g.W32 = W2; g.W16 = W2h; g.lr = lr; g.gout = sg ? gW2 : nullptr;
                g.A2 = dZ2lo;
                break;
            default:
                g = gdesc(GEMM_F16, EPI_SGD, 1, 1, D1, D0, B, dZ1, D1, X, D0, nullptr, D0);
                g.scale = bs; g.W32 = W1; g.W16 = W1h; g.lr = lr; g.gout = sg ? gW1 : nullptr;
                g.A2 = dZ1lo;
                break;
        }
        return g;
    }
    // Variant selection for the step's contractions (BEAM over the f16 kernels): each is timed with
    // its own epilogue (register pressure and epilogue traffic differ between epilogues), reading the
    // real operands, bias and activations but writing only to scratch, so tuning changes no
    // parameter, accumulator or activation.
    int tune() {
        // BEAM's disk cache (codegen/beam.go:118-169): with AH_GEMM_TUNE_CACHE naming a file, earlier
        // choices are loaded first and the file is rewritten after tuning.
        const char *cache = getenv("AH_GEMM_TUNE_CACHE");
        if (cache && *cache) {
            FILE *f = fopen(cache, "r");
            if (f) { fclose(f); int rc0 = ah_gemm_tune_cache(dev, cache, 0); if (rc0) return rc0; }
        }
        // AH_MLP3_VARIANTS="v0,...,v7" fixes the eight contractions' variants (0: tune that one), for
        // measurements of one choice against another
        const char *fixed = getenv("AH_MLP3_VARIANTS");
        if (fixed && *fixed) {
            const char *p = fixed;
            for (int i = 0; i < kGemms; i++) {
                char *end = nullptr;
                const long v = strtol(p, &end, 10);
                if (end == p || v < 0 || v > kGemm16Variants)
                    return set_error(AH_ERR_INVALID, "AH_MLP3_VARIANTS: 8 variants, 0..%d", kGemm16Variants);
                if (v) dev->gemm_variant[tune_key(gemm(i, false))] = (int)v;
                p = *end == ',' ? end + 1 : end;
            }
        }
        size_t most = 0;
        for (int i = 0; i < kGemms; i++) {
            GemmDesc g = gemm(i, false);
            most = std::max(most, (size_t)g.M * g.N);
        }
        half_t *s16 = nullptr;
        float *s32 = nullptr;
        int rc = AH_OK;
        if (hipMalloc(&s16, most * sizeof(half_t)) != hipSuccess || hipMalloc(&s32, most * sizeof(float)) != hipSuccess ||
            hipMemset(s32, 0, most * sizeof(float)) != hipSuccess)
            rc = set_error(AH_ERR_HIP, "MLP3: tuning scratch");
        bool fresh[kGemms] = {};
        for (int i = 0; i < kGemms && rc == AH_OK; i++) {
            GemmDesc g = gemm(i, false);
            if (dev->gemm_variant.count(tune_key(g))) continue;
            if (g.epi == EPI_SGD) {
                g.W32 = s32; g.W16 = s16; g.gout = nullptr;
            } else {
                // the partial sums (at most ceil(M/32) x N values) go to s32, which no other output uses
                g.C = s16;
                if (g.colsum) g.colsum = s32;
                if (g.lossacc) g.lossacc = s32;
            }
            rc = tune_gemm(dev, g, 4, nullptr, nullptr);
            fresh[i] = true;
        }
        hipFree(s16);
        hipFree(s32);
        if (rc == AH_OK) rc = refine(fresh);
        if (rc == AH_OK) rc = choose_pairs();
        if (rc == AH_OK) rc = clear_state();
        if (rc == AH_OK && cache && *cache) rc = ah_gemm_tune_cache(dev, cache, 1);
        return rc;
    }
    // Second BEAM stage: each contraction tuned above is re-timed inside the running step, every
    // variant in turn, and the fastest in place is kept. Timed alone, a variant sees its operands warm
    // from the previous launch and its epilogue rewriting scratch it just wrote; inside the step the
    // weight-update epilogues read master weights last touched a whole step earlier, which changes the
    // ranking (dW1 of config 3: the alone-fastest variant is 10% slower in place). The refinement runs
    // on hash-filled parameters and data before any slot is set; clear_state() zeroes them afterwards.
    // Contractions whose shape key another contraction of the step shares keep the choice from
    // timing alone (the probe brackets one launch, the key selects the variant for both).
    int refine(const bool *fresh) {
        std::string keys[kGemms];
        for (int i = 0; i < kGemms; i++) keys[i] = tune_key(gemm(i, false));
        bool any = false;
        for (int i = 0; i < kGemms; i++) any |= fresh[i];
        if (!any) return AH_OK;
        hipStream_t s = dev->stream;
        const float x_amp = 1.7320508f;
        AH_HIP(fill_hash(nullptr, X, (long)B * D0, 1u, x_amp, s));
        AH_HIP(fill_hash(nullptr, T, (long)B * D3, 2u, x_amp, s));
        AH_HIP(fill_hash(W1, W1h, (long)D1 * D0, 3u, x_amp / sqrtf((float)D0), s));
        AH_HIP(fill_hash(W2, W2h, (long)D2 * D1, 4u, x_amp / sqrtf((float)D1), s));
        AH_HIP(fill_hash(W3, W3h, (long)D3 * D2, 5u, x_amp / sqrtf((float)D2), s));
        AH_HIP(fill_hash(b1, b1h, D1, 6u, 0.01f, s));
        AH_HIP(fill_hash(b2, b2h, D2, 7u, 0.01f, s));
        AH_HIP(fill_hash(b3, b3h, D3, 8u, 0.01f, s));
        constexpr int kSteps = 4;
        int rc = AH_OK;
        const int saved = probe_index, saved_last = probe_last;
        const int saved_pairs[2] = {pair_v[0], pair_v[1]};
        pair_v[0] = pair_v[1] = 0;   // launch positions are those of the unpaired step
        auto steps = [&](int n) {
            for (int k = 0; k < n; k++) {
                launch_idx = 0;
                int r = enqueue(B, 0);
                if (r) return r;
            }
            return AH_OK;
        };
        rc = steps(2);
        for (int i = 0; i < kGemms && rc == AH_OK; i++) {
            if (!fresh[i]) continue;
            bool shared = false;
            for (int j = 0; j < kGemms; j++) shared |= j != i && keys[j] == keys[i];
            if (shared) continue;
            std::vector<double> t(kGemm16Variants + 1, 1e30);
            for (int pass = 0; pass < 2 && rc == AH_OK; pass++)
                for (int v = 1; v <= kGemm16Variants && rc == AH_OK; v++) {
                    dev->gemm_variant[keys[i]] = v;
                    if ((rc = steps(1))) break;   // the variant's first launch is not timed
                    probe_index = probe_last = kMlp3LaunchPos[i];
                    n_probe = 0;
                    rc = steps(kSteps);
                    probe_index = saved;
                    probe_last = saved_last;
                    double ms = 0.0;
                    int64_t n = 0;
                    if (rc == AH_OK) rc = ah_trainer_probe_read(this, &ms, &n);
                    if (rc == AH_OK && n > 0) t[v] = std::min(t[v], ms / n);
                }
            int bv = 1;
            for (int v = 2; v <= kGemm16Variants; v++)
                if (t[v] < t[bv]) bv = v;
            dev->gemm_variant[keys[i]] = bv;
        }
        probe_index = saved;
        probe_last = saved_last;
        pair_v[0] = saved_pairs[0];
        pair_v[1] = saved_pairs[1];
        n_probe = 0;
        launch_idx = 0;
        return rc;
    }
    // Partial-row stride of a column-sum epilogue: its waves start at row multiples of their tile height
    // (BM / WVM) and each stores the sum of its rows into row (first row / 32); with k-groups each group
    // finishes 32 rows. variant: the variant it runs with (0: the tuned or default choice).
    int colsum_stride(const GemmDesc &g, int variant) const {
        int v = variant;
        if (v == 0) {
            auto it = dev->gemm_variant.find(tune_key(g));
            v = it != dev->gemm_variant.end() ? it->second : gemm16_default_variant(g);
        }
        G16Params p;
        if (!gemm16_variant_params(v, &p) || p.kg > 1) return 1;
        return std::max(1, p.bm / p.wvm / 32);
    }
    // Paired launches: launched apart unless AH_PAIR_VARIANT fixes a pair variant, a tune cache holds a
    // choice, or AH_PAIR_TUNE=1 asks for timing. Timing runs whole steps with the two contractions
    // launched apart and paired with each pair variant (interleaved, three rounds, the best mean of 8
    // steps each), on hash-filled parameters and data, keeps the fastest and caches the choice under the
    // pair's key beside the variant choices. (Untimed by default: the paired launches have measured
    // slower in every alternating comparison, yet a noisy timing round could still pick them.)
    std::string pair_key(int q) const {
        const GemmDesc a = gemm(q == 0 ? 4 : 7, false), b = gemm(q == 0 ? 5 : 6, false);
        return "pair" + std::to_string(kPairSplit) + "/" + tune_key(a) + "/" + tune_key(b);
    }
    bool pair_admitted(int q) const {
        if (!pair_count || exact) return false;   // the paired kernels take one-plane operands
        const GemmDesc a = gemm(q == 0 ? 4 : 7, false), b = gemm(q == 0 ? 5 : 6, false);
        auto whole = [](const GemmDesc &g) { return g.M % 256 == 0 && g.N % 256 == 0 && g.K % 256 == 0; };
        return whole(a) && whole(b) && a.K % (64 * kPairSplit) == 0 &&
               (long)(a.M / 256) * (a.N / 256) * kPairSplit * 65536 <= pair_part_floats;
    }
    int choose_pairs() {
        // AH_PAIR_VARIANT fixes the choice (0: apart, 27 or 30: paired) without timing or caching it
        const char *force = getenv("AH_PAIR_VARIANT");
        if (force && *force) {
            const int v = atoi(force);
            if (v != 0 && v != 27 && v != 30) return set_error(AH_ERR_INVALID, "AH_PAIR_VARIANT must be 0, 27 or 30");
            for (int q = 0; q < 2; q++) pair_v[q] = pair_admitted(q) ? v : 0;
            return AH_OK;
        }
        bool todo[2];
        for (int q = 0; q < 2; q++) {
            auto it = dev->gemm_variant.find(pair_key(q));
            todo[q] = pair_admitted(q) && it == dev->gemm_variant.end();
            pair_v[q] = pair_admitted(q) && it != dev->gemm_variant.end() ? it->second : 0;
        }
        const char *tune = getenv("AH_PAIR_TUNE");
        if ((!todo[0] && !todo[1]) || !tune || strcmp(tune, "1") != 0) return AH_OK;
        hipStream_t s = dev->stream;
        const float x_amp = 1.7320508f;
        AH_HIP(fill_hash(nullptr, X, (long)B * D0, 1u, x_amp, s));
        AH_HIP(fill_hash(nullptr, T, (long)B * D3, 2u, x_amp, s));
        AH_HIP(fill_hash(W1, W1h, (long)D1 * D0, 3u, x_amp / sqrtf((float)D0), s));
        AH_HIP(fill_hash(W2, W2h, (long)D2 * D1, 4u, x_amp / sqrtf((float)D1), s));
        AH_HIP(fill_hash(W3, W3h, (long)D3 * D2, 5u, x_amp / sqrtf((float)D2), s));
        hipEvent_t e0, e1;
        AH_HIP(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence));
        AH_HIP(hipEventCreateWithFlags(&e1, hipEventDisableSystemFence));
        int rc = AH_OK;
        const int opts[3] = {0, 27, 30};
        for (int q = 0; q < 2 && rc == AH_OK; q++) {
            if (!todo[q]) continue;
            double best[3] = {1e30, 1e30, 1e30};
            for (int round = 0; round < 3 && rc == AH_OK; round++)
                for (int o = 0; o < 3 && rc == AH_OK; o++) {
                    pair_v[q] = opts[o];
                    for (int k = 0; k < 2 && rc == AH_OK; k++) { launch_idx = 0; rc = enqueue(B, 0); }
                    if (rc == AH_OK && hipEventRecord(e0, s) != hipSuccess) rc = set_error(AH_ERR_HIP, "MLP3: pair timing");
                    for (int k = 0; k < 8 && rc == AH_OK; k++) { launch_idx = 0; rc = enqueue(B, 0); }
                    float ms = 0.0f;
                    if (rc == AH_OK && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                                        hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
                        rc = set_error(AH_ERR_HIP, "MLP3: pair timing");
                    if (rc == AH_OK) best[o] = std::min(best[o], (double)ms);
                }
            int bo = 0;
            for (int o = 1; o < 3; o++)
                if (best[o] < best[bo]) bo = o;
            pair_v[q] = opts[bo];
            dev->gemm_variant[pair_key(q)] = opts[bo];
        }
        launch_idx = 0;
        hipEventDestroy(e0);
        hipEventDestroy(e1);
        return rc;
    }
    // Parameters, data, loss and accumulators all zero (the state create returns, tuned or not).
    int clear_state() {
        hipStream_t s = dev->stream;
        int rc = AH_OK;
        float *f32s[] = {W1, W2, W3, b1, b2, b3, loss};
        size_t nf[] = {(size_t)D1 * D0, (size_t)D2 * D1, (size_t)D3 * D2, (size_t)D1, (size_t)D2, (size_t)D3, 1};
        for (int k = 0; k < 7 && rc == AH_OK; k++)
            if (hipMemsetAsync(f32s[k], 0, nf[k] * 4, s) != hipSuccess) rc = set_error(AH_ERR_HIP, "MLP3: clearing state");
        half_t *f16s[] = {X, T, W1h, W2h, W3h, b1h, b2h, b3h};
        size_t nh[] = {(size_t)B * D0, (size_t)B * D3, (size_t)D1 * D0, (size_t)D2 * D1, (size_t)D3 * D2,
                       (size_t)D1, (size_t)D2, (size_t)D3};
        for (int k = 0; k < 8 && rc == AH_OK; k++)
            if (hipMemsetAsync(f16s[k], 0, nh[k] * 2, s) != hipSuccess) rc = set_error(AH_ERR_HIP, "MLP3: clearing state");
        if (rc == AH_OK && hipMemsetAsync(acc, 0, sizeof(float) * acc_floats(), s) != hipSuccess)
            rc = set_error(AH_ERR_HIP, "MLP3: clearing state");
        if (rc == AH_OK && hipStreamSynchronize(s) != hipSuccess) rc = set_error(AH_ERR_HIP, "MLP3: clearing state");
        return rc;
    }
    int enqueue(int64_t batch, int flags) override {
        if (batch != B) return set_error(AH_ERR_INVALID, "MLP3: batch %lld != %d", (long long)batch, B);
        hipStream_t s = dev->stream;
        const bool sg = flags & AH_STEP_STORE_GRADS;
        const float sc = (float)(1.0 / ((double)B * (double)D3));
        const float bs = 2.0f * sc;
        static const char *names[kGemms] = {"fc1", "fc2", "fc3_mse", "dH2", "dW3", "dH1", "dW2", "dW1"};
        if (!pair_v[0] && !pair_v[1]) {
            for (int i = 0; i < kGemms; i++) LAUNCH(names[kMlp3Order[i]], gemm_run(dev, gemm(kMlp3Order[i], sg), s));
        } else {
        for (int i = 0; i < 4; i++) LAUNCH(names[i], gemm_run(dev, gemm(i, sg), s));
        // dW3 beside dH1, then dW1 beside dW2 (each pair reads only finished inputs and writes
        // disjoint outputs)
        static constexpr int pairs[2][2] = {{4, 5}, {7, 6}};
        for (int q = 0; q < 2; q++) {
            const int a = pairs[q][0], b = pairs[q][1];
            if (pair_v[q]) {
                const GemmDesc ga = gemm(a, sg), gb = gemm(b, sg);
                hipError_t perr = hipSuccess;
                LAUNCH(q == 0 ? "dW3+dH1" : "dW1+dW2",
                       gemm16_pair_try_launch(ga, kPairSplit, &gb, pair_v[q], pair_count, pair_part, pair_part_floats,
                                              s, &perr) ? perr : hipErrorInvalidValue);
            } else {
                LAUNCH(names[a], gemm_run(dev, gemm(a, sg), s));
                LAUNCH(names[b], gemm_run(dev, gemm(b, sg), s));
            }
        }
        }
        TailArgs ta{};
        const int R = rblocks();
        // Each bias gradient's partial rows: one per 32-row block a wave of its producer starts (see
        // colsum_stride), stored (not accumulated) on every step, so the tail reads just those rows and
        // leaves them as they are.
        const int s3 = colsum_stride(gemm(2, false), 0), s2 = colsum_stride(gemm(3, false), 0);
        const int s1 = colsum_stride(gemm(5, false), pair_v[0]);
        ta.seg[0] = {b3, b3h, db3p(), sg ? gb3 : nullptr, D3, bs, (R + s3 - 1) / s3, (long)D3 * s3, 1};
        ta.seg[1] = {b2, b2h, db2p(), sg ? gb2 : nullptr, D2, bs, (R + s2 - 1) / s2, (long)D2 * s2, 1};
        ta.seg[2] = {b1, b1h, db1p(), sg ? gb1 : nullptr, D1, bs, (R + s1 - 1) / s1, (long)D1 * s1, 1};
        ta.nseg = 3; ta.lr = lr; ta.loss_mode = 1; ta.lossacc = lossp(); ta.loss_parts = R * lblocks();
        ta.loss_scale = sc; ta.loss_out = loss; ta.loss_sum = sg ? lsum : nullptr;
        LAUNCH("tail", step_tail(ta, s));
        return AH_OK;
    }
};

// ── config 5: movement + reduce chain ───────────────────────────────────────

struct ChainTrainer : ah_trainer {
    int R, Cc;
    float *X, *g, *dX, *dg, *work, *loss;
    int init() {
        R = (int)dims[0]; Cc = (int)dims[1];
        if (R <= 0 || Cc <= 0 || Cc % 4) return set_error(AH_ERR_INVALID, "CHAIN: need R > 0 and Cc %% 4 == 0");
        int rc = 0;
        rc |= alloc(&X, (size_t)R * Cc); rc |= alloc(&g, Cc); rc |= alloc(&dX, (size_t)R * Cc);
        rc |= alloc(&dg, Cc); rc |= alloc(&work, chain_workspace_floats(R, Cc)); rc |= alloc(&loss, 1);
        if (rc) return AH_ERR_HIP;
        AH_HIP(hipMemset(work, 0, sizeof(float) * chain_workspace_floats(R, Cc)));   // the arrival counter
        return AH_OK;
    }
    int max_batch() const override { return R; }
    int set(int slot, const void *h, int64_t n) override {
        if (slot == 0 && n == (int64_t)R * Cc) return copy_in(dev, X, h, (size_t)n * 4);
        if (slot == 1 && n == Cc) return copy_in(dev, g, h, (size_t)n * 4);
        return set_error(AH_ERR_INVALID, "CHAIN: bad set slot %d / size", slot);
    }
    int get(int slot, void *h, int64_t n) override {
        if (slot == 2 && n <= 1) return copy_out(dev, h, loss, 4);
        if (slot == 3 && n <= (int64_t)R * Cc) return copy_out(dev, h, dX, (size_t)n * 4);
        if (slot == 4 && n <= Cc) return copy_out(dev, h, dg, (size_t)n * 4);
        if (slot == 0 && n <= (int64_t)R * Cc) return copy_out(dev, h, X, (size_t)n * 4);
        return set_error(AH_ERR_INVALID, "CHAIN: bad get slot %d / size", slot);
    }
    int enqueue(int64_t, int) override {
        if (chain_resident_fits(R, Cc)) {   // each column strip held on chip: one pass over HBM
            LAUNCH("chain_resident", chain_step(X, g, R, Cc, work, dX, dg, loss, dev->stream, -1));
            return AH_OK;
        }
        LAUNCH("chain_stats", chain_step(X, g, R, Cc, work, dX, dg, loss, dev->stream, 0));
        LAUNCH("chain_finalize", chain_step(X, g, R, Cc, work, dX, dg, loss, dev->stream, 1));
        LAUNCH("chain_grad", chain_step(X, g, R, Cc, work, dX, dg, loss, dev->stream, 2));
        return AH_OK;
    }
};

// ── config 2: conv net ──────────────────────────────────────────────────────
// conv1(1->C1) ReLU pool2 -> conv2(C1->C2) ReLU pool2 -> flatten -> Linear(C2*(Hin/4)^2 -> NC) -> CE.

struct ConvNetTrainer : ah_trainer {
    int N, Hin, C1, C2, NC, P1, P2, F;
    float *x, *cw1, *cb1, *cw2, *cb2, *fw, *fb, *H1, *Pl1, *H2, *Pl2, *lg, *dlg, *dP2, *dZ2, *dP1, *dZ1;
    float *rowloss, *acc, *loss, *gcw1, *gcb1, *gcw2, *gcb2, *gfw, *gfb, *wpart1, *wpart2, *spart = nullptr, *sws = nullptr;
    int32_t *lab;
    bool fused = false;   // the sample-parallel forward and backward kernels (convnet.h) + the tail
    int init() {
        N = (int)dims[0]; Hin = (int)dims[1]; C1 = (int)dims[2]; C2 = (int)dims[3]; NC = (int)dims[4];
        if (N <= 0 || Hin <= 0 || Hin % 4 || C1 <= 0 || C2 <= 0 || NC <= 0) return set_error(AH_ERR_INVALID, "CONVNET: bad dims");
        P1 = Hin / 2; P2 = Hin / 4; F = C2 * P2 * P2;
        int rc = 0;
        rc |= alloc(&x, (size_t)N * Hin * Hin); rc |= alloc(&lab, N);
        rc |= alloc(&cw1, (size_t)C1 * 9); rc |= alloc(&cb1, C1); rc |= alloc(&cw2, (size_t)C2 * C1 * 9); rc |= alloc(&cb2, C2);
        rc |= alloc(&fw, (size_t)NC * F); rc |= alloc(&fb, NC);
        rc |= alloc(&H1, (size_t)N * C1 * Hin * Hin); rc |= alloc(&Pl1, (size_t)N * C1 * P1 * P1);
        rc |= alloc(&H2, (size_t)N * C2 * P1 * P1); rc |= alloc(&Pl2, (size_t)N * F);
        rc |= alloc(&lg, (size_t)N * NC); rc |= alloc(&dlg, (size_t)N * NC); rc |= alloc(&dP2, (size_t)N * F);
        rc |= alloc(&dZ2, (size_t)N * C2 * P1 * P1); rc |= alloc(&dP1, (size_t)N * C1 * P1 * P1);
        rc |= alloc(&dZ1, (size_t)N * C1 * Hin * Hin); rc |= alloc(&rowloss, N); rc |= alloc(&acc, NC);
        rc |= alloc(&loss, 1); rc |= alloc(&gcw1, (size_t)C1 * 9); rc |= alloc(&gcb1, C1);
        rc |= alloc(&wpart1, (size_t)conv_bwd_w_splits(N, 1, Hin, C1) * C1 * 10);
        rc |= alloc(&wpart2, (size_t)conv_bwd_w_splits(N, C1, P1, C2) * C2 * C1 * 10);
        rc |= alloc(&gcw2, (size_t)C2 * C1 * 9); rc |= alloc(&gcb2, C2); rc |= alloc(&gfw, (size_t)NC * F); rc |= alloc(&gfb, NC);
        fused = convnet_fused_ok(Hin, C1, C2, NC);
        if (fused) rc |= alloc(&spart, (size_t)N * net_part(Hin, C1, C2, NC).total);
        if (fused) rc |= alloc(&sws, (size_t)convnet_fused_ws_floats(N, Hin, C1, C2, NC));
        if (rc) return AH_ERR_HIP;
        AH_HIP(hipMemset(acc, 0, sizeof(float) * NC));
        return AH_OK;
    }
    struct Slot { void *p; int64_t n; };
    Slot slot_of(int i) {
        Slot t[] = {{x, (int64_t)N * Hin * Hin}, {lab, N}, {cw1, (int64_t)C1 * 9}, {cb1, C1}, {cw2, (int64_t)C2 * C1 * 9},
                    {cb2, C2}, {fw, (int64_t)NC * F}, {fb, NC}, {loss, 1}, {gcw1, (int64_t)C1 * 9}, {gcb1, C1},
                    {gcw2, (int64_t)C2 * C1 * 9}, {gcb2, C2}, {gfw, (int64_t)NC * F}, {gfb, NC}};
        return (i >= 0 && i < 15) ? t[i] : Slot{nullptr, 0};
    }
    int set(int slot, const void *h, int64_t n) override {
        if (slot < 0 || slot > 7) return set_error(AH_ERR_INVALID, "CONVNET: slot %d not settable", slot);
        Slot t = slot_of(slot);
        if (n > t.n) return set_error(AH_ERR_INVALID, "CONVNET: slot %d too large", slot);
        return copy_in(dev, t.p, h, (size_t)n * 4);
    }
    int get(int slot, void *h, int64_t n) override {
        Slot t = slot_of(slot);
        if (!t.p || n > t.n) return set_error(AH_ERR_INVALID, "CONVNET: bad get slot %d", slot);
        return copy_out(dev, h, t.p, (size_t)n * 4);
    }
    int enqueue(int64_t batch, int flags) override {
        const int B = (int)batch;
        hipStream_t s = dev->stream;
        const bool sg = flags & AH_STEP_STORE_GRADS;
        const float a = (float)(-1.0 / (double)B);
        if (fused) {
            LAUNCH("convnet_fwd", convnet_fwd_fused(x, cw1, cb1, cw2, cb2, fw, B, Hin, C1, C2, NC, sws, s));
            LAUNCH("convnet_bwd", convnet_bwd_fused(x, lab, cw2, fw, fb, B, Hin, C1, C2, NC, a, sws, rowloss, spart, s));
            const NetPart o = net_part(Hin, C1, C2, NC);
            TailArgs ta{};
            float *p[6] = {cw1, cb1, cw2, cb2, fw, fb}, *go[6] = {gcw1, gcb1, gcw2, gcb2, gfw, gfb};
            const long off[6] = {o.cw1, o.cb1, o.cw2, o.cb2, o.fw, o.fb};
            const long len[6] = {o.cb1 - o.cw1, o.cw2 - o.cb1, o.cb2 - o.cw2, o.fw - o.cb2, o.fb - o.fw, o.total - o.fb};
            for (int i = 0; i < 6; i++) ta.seg[i] = {p[i], nullptr, spart + off[i], sg ? go[i] : nullptr, len[i], 1.0f, B, o.total, 1};
            ta.nseg = 6; ta.lr = lr; ta.loss_mode = 2; ta.loss_scale = a; ta.rowloss = rowloss; ta.nrow = B; ta.loss_out = loss;
            LAUNCH("tail", step_tail(ta, s));
            return AH_OK;
        }
        LAUNCH("conv1", conv_fwd_relu_pool(x, B, 1, Hin, cw1, cb1, C1, H1, Pl1, s));
        LAUNCH("conv2", conv_fwd_relu_pool(Pl1, B, C1, P1, cw2, cb2, C2, H2, Pl2, s));
        GemmDesc g = gdesc(GEMM_F32, EPI_BIAS, 0, 0, B, NC, F, Pl2, F, fw, F, lg, NC);
        g.bias = fb;
        LAUNCH("fc", gemm_run(dev, g, s));
        LAUNCH("softmax_ce", softmax_ce(lg, lab, B, NC, a, dlg, rowloss, s));
        LAUNCH("dfb", colsum_add(dlg, B, NC, NC, acc, s));
        g = gdesc(GEMM_F32, EPI_STORE, 0, 1, B, F, NC, dlg, NC, fw, F, dP2, F);
        LAUNCH("dP2", gemm_run(dev, g, s));
        g = gdesc(GEMM_F32, EPI_SGD, 1, 1, NC, F, B, dlg, NC, Pl2, F, nullptr, F);
        g.W32 = fw; g.lr = lr; g.gout = sg ? gfw : nullptr;
        LAUNCH("dfw", gemm_run(dev, g, s));
        LAUNCH("pool2_bwd", pool_relu_bwd(dP2, H2, Pl2, B * C2, P1, dZ2, s));
        LAUNCH("conv2_dx", conv_bwd_x(dZ2, cw2, B, C1, P1, C2, dP1, s));
        LAUNCH("conv2_dw", conv_bwd_w_partial(Pl1, dZ2, B, C1, P1, C2, wpart2, s));
        LAUNCH("conv2_dw_sgd", conv_bwd_w_finalize(wpart2, B, C1, P1, C2, cw2, cb2, lr, sg ? gcw2 : nullptr, sg ? gcb2 : nullptr, s));
        LAUNCH("pool1_bwd", pool_relu_bwd(dP1, H1, Pl1, B * C1, Hin, dZ1, s));
        LAUNCH("conv1_dw", conv_bwd_w_partial(x, dZ1, B, 1, Hin, C1, wpart1, s));
        LAUNCH("conv1_dw_sgd", conv_bwd_w_finalize(wpart1, B, 1, Hin, C1, cw1, cb1, lr, sg ? gcw1 : nullptr, sg ? gcb1 : nullptr, s));
        TailArgs ta{};
        ta.seg[0] = {fb, nullptr, acc, sg ? gfb : nullptr, NC, 1.0f};
        ta.nseg = 1; ta.lr = lr; ta.loss_mode = 2; ta.loss_scale = a; ta.rowloss = rowloss; ta.nrow = B; ta.loss_out = loss;
        LAUNCH("tail", step_tail(ta, s));
        return AH_OK;
    }
};

// ── C ABI ───────────────────────────────────────────────────────────────────

extern "C" {

int ah_trainer_create(ah_device *dev, int32_t kind, const int64_t *dims, int32_t n_dims, float lr, ah_trainer **out) {
    if (!dev || !dims || !out) return set_error(AH_ERR_INVALID, "ah_trainer_create: null argument");
    hipSetDevice(dev->ordinal);
    ah_trainer *t = nullptr;
    int rc = AH_OK;
    auto setup = [&](ah_trainer *tt, int need, int optional = 0) {
        tt->dev = dev; tt->kind = kind; tt->lr = lr;
        if (n_dims < need || n_dims > need + optional)
            return set_error(AH_ERR_INVALID, "kind %d needs %d dims, got %d", kind, need, n_dims);
        tt->dims.assign(dims, dims + n_dims);
        return AH_OK;
    };
    switch (kind) {
        case AH_TRAIN_MLP_CE: { auto *m = new MlpCeTrainer(); t = m; rc = setup(t, 4); if (!rc) rc = m->init(); break; }
        case AH_TRAIN_MLP3_F16: { auto *m = new Mlp3Trainer(); t = m; rc = setup(t, 5, 1); if (!rc) rc = m->init(); break; }
        case AH_TRAIN_CHAIN: { auto *m = new ChainTrainer(); t = m; rc = setup(t, 2); if (!rc) rc = m->init(); break; }
        case AH_TRAIN_CONVNET: { auto *m = new ConvNetTrainer(); t = m; rc = setup(t, 5); if (!rc) rc = m->init(); break; }
        default: return set_error(AH_ERR_INVALID, "ah_trainer_create: unknown kind %d", kind);
    }
    if (rc != AH_OK) { delete t; return rc; }
    *out = t;
    return AH_OK;
}

void ah_trainer_destroy(ah_trainer *t) { delete t; }

int ah_trainer_set(ah_trainer *t, int32_t slot, const void *host, int64_t n) {
    if (!t || !host) return set_error(AH_ERR_INVALID, "ah_trainer_set: null argument");
    return t->set(slot, host, n);
}
int ah_trainer_get(ah_trainer *t, int32_t slot, void *host, int64_t n) {
    if (!t || !host) return set_error(AH_ERR_INVALID, "ah_trainer_get: null argument");
    return t->get(slot, host, n);
}

// Replays `steps` consecutive steps as one hipGraph launch. One graph per (batch, gradient-output
// choice, step count), captured on first use: the gradient outputs change kernels' arguments, and a
// graph of several steps holds that many copies of the step's kernel sequence. A hipGraphLaunch costs
// this runtime about 17 us of host time and about 4.5 us of GPU idle time per launch whatever the graph
// holds (measured on MI355X with 1-6 short kernels per graph), so a graph of k steps pays that once per k.
static int graph_steps(ah_trainer *t, int64_t batch, int32_t flags, int steps) {
    const int64_t key = ((batch * 2 + ((flags & AH_STEP_STORE_GRADS) ? 1 : 0)) << 6) | steps;
    auto it = t->graphs.find(key);
    if (it == t->graphs.end()) {
        int saved = t->probe_index;
        t->probe_index = -1;
        int rc = ah_graph_begin(t->dev);
        if (rc) { t->probe_index = saved; return rc; }
        int rc2 = AH_OK;
        for (int i = 0; i < steps && rc2 == AH_OK; i++) {
            t->launch_idx = 0;
            rc2 = t->enqueue(batch, flags & ~AH_STEP_GRAPH);
        }
        ah_graph *g = nullptr;
        rc = ah_graph_end(t->dev, &g);
        t->probe_index = saved;
        if (rc2) { ah_graph_destroy(g); return rc2; }
        if (rc) return rc;
        it = t->graphs.emplace(key, g).first;
    }
    return ah_graph_replay(t->dev, it->second);
}

int ah_trainer_step(ah_trainer *t, int64_t batch, int32_t flags) {
    if (!t) return set_error(AH_ERR_INVALID, "ah_trainer_step: null trainer");
    if (batch <= 0 || batch > t->max_batch())
        return set_error(AH_ERR_INVALID, "ah_trainer_step: batch %lld outside [1, %d]", (long long)batch, t->max_batch());
    if (int rc = t->prepare(batch)) return rc;
    if (flags & AH_STEP_GRAPH) return graph_steps(t, batch, flags, 1);
    t->launch_idx = 0;
    return t->enqueue(batch, flags);
}

int ah_trainer_steps(ah_trainer *t, int64_t batch, int32_t flags, int32_t n) {
    if (!t) return set_error(AH_ERR_INVALID, "ah_trainer_steps: null trainer");
    if (n < 0) return set_error(AH_ERR_INVALID, "ah_trainer_steps: n = %d", n);
    if (batch <= 0 || batch > t->max_batch())
        return set_error(AH_ERR_INVALID, "ah_trainer_steps: batch %lld outside [1, %d]", (long long)batch, t->max_batch());
    if (n == 0) return AH_OK;
    if (int rc = t->prepare(batch)) return rc;
    if (!(flags & AH_STEP_GRAPH)) {
        for (int32_t i = 0; i < n; i++) {
            t->launch_idx = 0;
            if (int rc = t->enqueue(batch, flags)) return rc;
        }
        return AH_OK;
    }
    // whole graphs of kMaxGraphSteps steps, then one graph of the remainder
    for (int32_t done = 0; done < n;) {
        const int u = std::min<int32_t>(kMaxGraphSteps, n - done);
        if (int rc = graph_steps(t, batch, flags, u)) return rc;
        done += u;
    }
    return AH_OK;
}

int ah_trainer_probe(ah_trainer *t, int32_t kernel_index) {
    if (!t) return set_error(AH_ERR_INVALID, "ah_trainer_probe: null trainer");
    t->probe_index = t->probe_last = kernel_index < 0 ? -1 : kernel_index;
    t->n_probe = 0;
    return AH_OK;
}

int ah_trainer_probe_span(ah_trainer *t, int32_t first, int32_t last) {
    if (!t) return set_error(AH_ERR_INVALID, "ah_trainer_probe_span: null trainer");
    if (first < 0 || last < first - 1)
        return set_error(AH_ERR_INVALID, "ah_trainer_probe_span: span [%d, %d]", first, last);
    t->probe_index = first;
    t->probe_last = last;
    t->n_probe = 0;
    return AH_OK;
}

int ah_trainer_probe_read(ah_trainer *t, double *total_ms, int64_t *count) {
    if (!t || !total_ms || !count) return set_error(AH_ERR_INVALID, "ah_trainer_probe_read: null argument");
    AH_HIP(hipStreamSynchronize(t->dev->stream));
    double tot = 0.0;
    for (size_t i = 0; i < t->n_probe; i++) {
        float ms = 0.0f;
        AH_HIP(hipEventElapsedTime(&ms, t->ev_a[i], t->ev_b[i]));
        tot += ms;
    }
    *total_ms = tot;
    *count = (int64_t)t->n_probe;
    t->n_probe = 0;
    return AH_OK;
}

int ah_trainer_kernel_count(ah_trainer *t, int64_t batch, int32_t *count) {
    if (!t || !count) return set_error(AH_ERR_INVALID, "ah_trainer_kernel_count: null argument");
    // Count by a dry enqueue into a capture that is then discarded.
    int saved = t->probe_index;
    t->probe_index = -1;
    int rc = ah_graph_begin(t->dev);
    if (rc) return rc;
    t->launch_idx = 0;
    t->names.clear();
    t->record_names = true;
    int rc2 = t->enqueue(batch, 0);
    t->record_names = false;
    ah_graph *g = nullptr;
    rc = ah_graph_end(t->dev, &g);
    ah_graph_destroy(g);
    t->probe_index = saved;
    if (rc2) return rc2;
    if (rc) return rc;
    *count = t->launch_idx;
    return AH_OK;
}

int ah_trainer_kernel_name(ah_trainer *t, int32_t index, char *buf, int32_t cap) {
    if (!t || !buf || cap <= 0) return set_error(AH_ERR_INVALID, "ah_trainer_kernel_name: null argument");
    if (index < 0 || index >= (int32_t)t->names.size())
        return set_error(AH_ERR_INVALID, "ah_trainer_kernel_name: index %d outside the %d launches counted", (int)index,
                         (int)t->names.size());
    snprintf(buf, (size_t)cap, "%s", t->names[index].c_str());
    return AH_OK;
}

// Direct kernel entry points ---------------------------------------------------

int ah_gemm(ah_device *dev, const ah_gemm_desc *d) {
    if (!dev || !d) return set_error(AH_ERR_INVALID, "ah_gemm: null argument");
    if (d->dtype != AH_F32 && d->dtype != AH_F16) return set_error(AH_ERR_UNSUPPORTED, "ah_gemm: dtype %d", d->dtype);
    if (d->M < 0 || d->N < 0 || d->K < 0 || !d->A || !d->B) return set_error(AH_ERR_INVALID, "ah_gemm: bad shape/pointer");
    if (d->epi == AH_EPI_SGD ? !d->W32 : !d->C) return set_error(AH_ERR_INVALID, "ah_gemm: missing output");
    if ((d->epi == AH_EPI_BIAS || d->epi == AH_EPI_BIAS_RELU || d->epi == AH_EPI_MSE) && !d->bias)
        return set_error(AH_ERR_INVALID, "ah_gemm: epilogue needs bias");
    if ((d->epi == AH_EPI_MASK || d->epi == AH_EPI_MSE) && !d->aux) return set_error(AH_ERR_INVALID, "ah_gemm: epilogue needs aux");
    if (d->epi == AH_EPI_MSE && (d->dtype != AH_F16 || !d->lossacc)) return set_error(AH_ERR_INVALID, "ah_gemm: MSE epilogue is f16 with lossacc");
    if (d->tile != 0 && d->tile != 64 && d->tile != 128 && d->tile != 256) return set_error(AH_ERR_INVALID, "ah_gemm: tile %d", d->tile);
    if (d->variant < 0 || d->variant > kGemm16Variants) return set_error(AH_ERR_INVALID, "ah_gemm: variant %d", d->variant);
    GemmDesc g;
    memset(&g, 0, sizeof g);
    g.dtype = d->dtype == AH_F16 ? GEMM_F16 : GEMM_F32;
    g.epi = d->epi; g.ta = d->ta; g.tb = d->tb; g.M = d->M; g.N = d->N; g.K = d->K;
    g.A = d->A; g.B = d->B; g.lda = d->lda; g.ldb = d->ldb; g.C = d->C; g.ldc = d->ldc; g.bias = d->bias;
    g.aux = d->aux; g.ldaux = d->ldaux; g.scale = d->scale; g.colsum = d->colsum; g.W32 = d->W32; g.W16 = d->W16;
    g.lr = d->lr; g.gout = d->gout; g.lossacc = d->lossacc; g.tile = d->tile; g.variant = d->variant;
    AH_HIP(gemm_run(dev, g, dev->stream));
    return AH_OK;
}

int ah_gemm_tune_cache(ah_device *dev, const char *path, int32_t save) {
    if (!dev || !path) return set_error(AH_ERR_INVALID, "ah_gemm_tune_cache: null argument");
    if (save) {
        FILE *f = fopen(path, "w");
        if (!f) return set_error(AH_ERR_INVALID, "gemm tune cache: cannot write %s", path);
        std::vector<std::pair<std::string, int>> rows(dev->gemm_variant.begin(), dev->gemm_variant.end());
        std::sort(rows.begin(), rows.end());
        fprintf(f, "# anneal_hip gemm variants v1 %s\n", dev->arch.c_str());
        for (auto &r : rows) fprintf(f, "%s %d\n", r.first.c_str(), r.second);
        if (fclose(f) != 0) return set_error(AH_ERR_INVALID, "gemm tune cache: write to %s failed", path);
        return AH_OK;
    }
    FILE *f = fopen(path, "r");
    if (!f) return set_error(AH_ERR_INVALID, "gemm tune cache: cannot read %s", path);
    char line[256];
    int rc = AH_OK, lineno = 0;
    std::unordered_map<std::string, int> got;
    while (fgets(line, sizeof line, f)) {
        lineno++;
        if (line[0] == '#' || line[0] == '\n') {
            // the header names the device the choices were timed on; another arch starts afresh
            if (lineno == 1 && !strstr(line, dev->arch.c_str())) { fclose(f); return AH_OK; }
            continue;
        }
        char key[128];
        int v = 0;
        const bool parsed = sscanf(line, "%127s %d", key, &v) == 2;
        const bool pair = parsed && strncmp(key, "pair", 4) == 0;
        const bool f32 = parsed && strncmp(key, "0/", 2) == 0;   // tune_key: dtype first
        const bool ok = pair ? (v == 0 || v == 27 || v == 30)
                        : f32 ? v >= 0 && v < (int)f32_cfgs().size() : v >= 1 && v <= kGemm16Variants;
        if (sscanf(line, "%127s %d", key, &v) != 2 || !ok) {
            rc = set_error(AH_ERR_INVALID, "gemm tune cache %s: bad line %d", path, lineno);
            break;
        }
        got[key] = v;
    }
    fclose(f);
    if (rc == AH_OK)
        for (auto &kv : got) dev->gemm_variant[kv.first] = kv.second;
    return rc;
}

int ah_gemm_tune(ah_device *dev, const ah_gemm_desc *d, int32_t iterations, int32_t *best_variant, double *best_us) {
    if (!dev || !d) return set_error(AH_ERR_INVALID, "ah_gemm_tune: null argument");
    if (d->dtype != AH_F16 && d->dtype != AH_F32) return set_error(AH_ERR_UNSUPPORTED, "ah_gemm_tune: f16 and f32 contractions only");
    if (d->M <= 0 || d->N <= 0 || d->K <= 0 || !d->A || !d->B) return set_error(AH_ERR_INVALID, "ah_gemm_tune: bad shape/pointer");
    if (d->epi == AH_EPI_SGD ? !d->W32 : !d->C) return set_error(AH_ERR_INVALID, "ah_gemm_tune: missing output");
    GemmDesc g;
    memset(&g, 0, sizeof g);
    g.dtype = d->dtype == AH_F16 ? GEMM_F16 : GEMM_F32;
    g.epi = d->epi; g.ta = d->ta; g.tb = d->tb; g.M = d->M; g.N = d->N; g.K = d->K;
    g.A = d->A; g.B = d->B; g.lda = d->lda; g.ldb = d->ldb; g.C = d->C; g.ldc = d->ldc; g.bias = d->bias;
    g.aux = d->aux; g.ldaux = d->ldaux; g.scale = d->scale; g.colsum = d->colsum; g.W32 = d->W32; g.W16 = d->W16;
    g.lr = d->lr; g.gout = d->gout; g.lossacc = d->lossacc;
    int bv = 0;
    int rc = tune_gemm(dev, g, iterations, &bv, best_us);
    if (rc == AH_OK && best_variant) *best_variant = bv;
    return rc;
}

int ah_softmax_ce(ah_device *dev, const float *z, const int32_t *labels, int32_t B, int32_t C, float *dz, float *loss) {
    if (!dev || !z || !labels || !dz || !loss || B <= 0 || C <= 0) return set_error(AH_ERR_INVALID, "ah_softmax_ce: bad argument");
    float *rl = nullptr;
    AH_HIP(hipMalloc(&rl, (size_t)B * 4));
    float a = (float)(-1.0 / (double)B);
    hipError_t e = softmax_ce(z, labels, B, C, a, dz, rl, dev->stream);
    if (e == hipSuccess) e = sum_scale(rl, B, a, loss, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    hipFree(rl);
    if (e != hipSuccess) return fail_hip(e, "ah_softmax_ce");
    return AH_OK;
}

int ah_chain_step(ah_device *dev, const float *X, const float *g, int32_t R, int32_t Cc, float *dX, float *dg, float *loss) {
    if (!dev || !X || !g || !dX || !dg || !loss || R <= 0 || Cc <= 0 || Cc % 4)
        return set_error(AH_ERR_INVALID, "ah_chain_step: bad argument (Cc must be a multiple of 4)");
    float *w = nullptr;
    AH_HIP(hipMalloc(&w, (size_t)chain_workspace_floats(R, Cc) * 4));
    hipError_t e = hipMemsetAsync(w, 0, 256, dev->stream);   // the resident path's arrival counter
    if (e == hipSuccess) e = chain_step(X, g, R, Cc, w, dX, dg, loss, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    hipFree(w);
    if (e != hipSuccess) return fail_hip(e, "ah_chain_step");
    return AH_OK;
}

int ah_chain_step_noalloc(ah_device *dev, const float *X, const float *g, int32_t R, int32_t Cc, float *dX, float *dg,
                          float *loss) {
    if (!dev || !X || !g || !dX || !dg || !loss || R <= 0 || Cc <= 0 || Cc % 4)
        return set_error(AH_ERR_INVALID, "ah_chain_step_noalloc: bad argument (Cc must be a multiple of 4)");
    const long need = chain_workspace_floats(R, Cc), cap = chain_scratch_floats();
    if (need > cap)
        return set_error(AH_ERR_INVALID, "ah_chain_step_noalloc: R=%d x Cc=%d needs %ld workspace floats, the maximum is %ld",
                         R, Cc, need, cap);
    if (!dev->chain_scratch) return set_error(AH_ERR_INVALID, "ah_chain_step_noalloc: device has no chain workspace");
    AH_HIP(chain_step(X, g, R, Cc, dev->chain_scratch, dX, dg, loss, dev->stream));
    return AH_OK;
}

}  // extern "C"
