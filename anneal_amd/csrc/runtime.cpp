// runtime.cpp — device, buffers, dtype codec, hiprtc module cache, launches and graphs.
//
// The reference allocates, uploads, compiles and releases everything inside every Run
// (backend/webgpu/executor.go:80-237). Here a device owns one HIP stream for its lifetime, modules are
// compiled once per source hash, and buffers are explicit so callers can keep them resident.
#include <hip/hiprtc.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "ah_internal.h"
#include "rowops.h"
#include "gemm.h"

namespace ah {

static thread_local std::string g_err;

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int fail_hip(hipError_t e, const char *what) {
    return set_error(AH_ERR_HIP, "hip: %s failed: %s", what, hipGetErrorString(e));
}

int64_t dtype_bytes(int32_t dtype) { return dtype == AH_F16 ? 2 : 4; }

}  // namespace ah

using namespace ah;

extern "C" {

const char *ah_last_error(void) { return g_err.c_str(); }

// ── codec: uop/dtype.go:392-487 ─────────────────────────────────────────────

uint16_t ah_f32_to_f16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)(bits >> 31);
    int32_t exp = (int32_t)((bits >> 23) & 0xFF) - 127;
    uint32_t frac = bits & 0x7FFFFF;
    if (exp == 128) {
        if (frac) {
            uint16_t m = (uint16_t)(frac >> 13);
            return (uint16_t)((sign << 15) | 0x7C00 | (m ? m : 1));
        }
        return (uint16_t)((sign << 15) | 0x7C00);
    }
    if (exp > 15) return (uint16_t)((sign << 15) | 0x7C00);
    if (exp < -25) return (uint16_t)(sign << 15);
    if (exp < -14) {
        uint32_t m = frac | 0x800000, sh = (uint32_t)(-1 - exp);
        uint32_t r = m >> (sh - 1);
        if ((r & 1) && ((r & 2) || (m & ((1u << (sh - 1)) - 1)))) r += 2;
        return (uint16_t)((sign << 15) | (uint16_t)(r >> 1));
    }
    uint32_t r = frac >> 12;
    if ((r & 1) && ((r & 2) || (frac & 0xFFF))) r += 2;
    uint16_t m16 = (uint16_t)(r >> 1);
    int32_t e16 = exp + 15;
    if (m16 & 0x400) { m16 &= 0x3FF; e16++; }
    if (e16 > 30) return (uint16_t)((sign << 15) | 0x7C00);
    return (uint16_t)((sign << 15) | ((uint16_t)e16 << 10) | m16);
}

float ah_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1F, frac = h & 0x3FF, bits;
    if (exp == 0) {
        if (!frac) bits = sign;
        else {
            uint32_t e = 127 - 14;
            while (!(frac & 0x400)) { frac <<= 1; e--; }
            bits = sign | (e << 23) | ((frac & 0x3FF) << 13);
        }
    } else if (exp == 31) bits = sign | 0x7F800000 | (frac << 13);
    else bits = sign | ((exp + 112) << 23) | (frac << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// ── device ──────────────────────────────────────────────────────────────────

int ah_open(int ordinal, ah_device **out) {
    if (!out) return set_error(AH_ERR_INVALID, "ah_open: null out");
    int n = 0;
    AH_HIP(hipGetDeviceCount(&n));
    if (ordinal < 0 || ordinal >= n) return set_error(AH_ERR_INVALID, "ah_open: ordinal %d of %d devices", ordinal, n);
    AH_HIP(hipSetDevice(ordinal));
    ah_device *d = new ah_device();
    d->ordinal = ordinal;
    hipError_t e = hipGetDeviceProperties(&d->props, ordinal);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete d;
        return fail_hip(e, "ah_open");
    }
    d->arch = d->props.gcnArchName;
    if (d->arch.rfind("gfx950", 0) != 0) {
        hipStreamDestroy(d->stream);
        delete d;
        return set_error(AH_ERR_UNSUPPORTED, "ah_open: device arch %s is not gfx950", d->props.gcnArchName);
    }
    e = chain_scratch_init(ordinal, &d->chain_scratch);   // the device is current (hipSetDevice above)
    if (e != hipSuccess) {
        hipStreamDestroy(d->stream);
        delete d;
        return fail_hip(e, "ah_open: chain workspace address");
    }
    {   // split-K counters start at zero; the kernels leave them at zero
        const size_t sync_bytes = (size_t)kSplitKMaxTiles * 2 * sizeof(int);
        e = hipMalloc(&d->splitk_ws, sync_bytes + (size_t)kSplitKPartFloats * sizeof(float));
        if (e == hipSuccess) e = hipMemset(d->splitk_ws, 0, sync_bytes);
        if (e != hipSuccess) {
            if (d->splitk_ws) hipFree(d->splitk_ws);
            hipStreamDestroy(d->stream);
            delete d;
            return fail_hip(e, "ah_open: split-K workspace");
        }
    }
    *out = d;
    return AH_OK;
}

void ah_close(ah_device *d) {
    if (!d) return;
    hipSetDevice(d->ordinal);
    hipStreamSynchronize(d->stream);
    for (auto &kv : d->modules) {
        if (kv.second->module) hipModuleUnload(kv.second->module);
        delete kv.second->tmpl;
        delete kv.second;
    }
    if (d->splitk_ws) hipFree(d->splitk_ws);
    if (d->t0) hipEventDestroy(d->t0);
    if (d->t1) hipEventDestroy(d->t1);
    hipStreamDestroy(d->stream);
    delete d;
}

int ah_get_caps(ah_device *d, ah_caps *out) {
    if (!d || !out) return set_error(AH_ERR_INVALID, "ah_get_caps: null argument");
    memset(out, 0, sizeof *out);
    out->has_f16 = 1;
    out->has_bf16 = 1;
    out->cu_count = d->props.multiProcessorCount;
    out->wavefront = d->props.warpSize;
    out->hbm_bytes = (int64_t)d->props.totalGlobalMem;
    out->lds_bytes_per_block = (int64_t)d->props.sharedMemPerBlock;
    snprintf(out->arch, sizeof out->arch, "%s", d->props.gcnArchName);
    return AH_OK;
}

int ah_sync(ah_device *d) {
    if (!d) return set_error(AH_ERR_INVALID, "ah_sync: null device");
    AH_HIP(hipStreamSynchronize(d->stream));
    return AH_OK;
}

// ── buffers ─────────────────────────────────────────────────────────────────

int ah_buf_alloc(ah_device *d, int64_t n, int32_t dtype, void **dptr) {
    if (!d || !dptr || n < 0) return set_error(AH_ERR_INVALID, "ah_buf_alloc: bad argument");
    size_t bytes = (size_t)(n ? n : 1) * (size_t)dtype_bytes(dtype);
    hipError_t e = hipMalloc(dptr, bytes);
    if (e == hipErrorOutOfMemory) return set_error(AH_ERR_NOMEM, "ah_buf_alloc: %zu bytes: out of memory", bytes);
    if (e != hipSuccess) return fail_hip(e, "hipMalloc");
    return AH_OK;
}

int ah_buf_free(ah_device *d, void *p) {
    if (!d) return set_error(AH_ERR_INVALID, "ah_buf_free: null device");
    if (p) AH_HIP(hipFree(p));
    return AH_OK;
}

int ah_upload(ah_device *d, void *dptr, const float *src, int64_t n, int32_t dtype) {
    if (!d || !dptr || (!src && n)) return set_error(AH_ERR_INVALID, "ah_upload: bad argument");
    if (dtype == AH_F16) {
        std::vector<uint16_t> h((size_t)n);
        for (int64_t i = 0; i < n; i++) h[i] = ah_f32_to_f16(src[i]);
        AH_HIP(hipMemcpyAsync(dptr, h.data(), (size_t)n * 2, hipMemcpyHostToDevice, d->stream));
        AH_HIP(hipStreamSynchronize(d->stream));
    } else if (dtype == AH_BF16) {
        std::vector<uint32_t> h((size_t)n);
        for (int64_t i = 0; i < n; i++) { uint32_t b; memcpy(&b, &src[i], 4); h[i] = b & 0xFFFF0000u; }
        AH_HIP(hipMemcpyAsync(dptr, h.data(), (size_t)n * 4, hipMemcpyHostToDevice, d->stream));
        AH_HIP(hipStreamSynchronize(d->stream));
    } else {
        AH_HIP(hipMemcpyAsync(dptr, src, (size_t)n * 4, hipMemcpyHostToDevice, d->stream));
        AH_HIP(hipStreamSynchronize(d->stream));
    }
    return AH_OK;
}

int ah_download(ah_device *d, float *dst, const void *dptr, int64_t n, int32_t dtype) {
    if (!d || !dptr || (!dst && n)) return set_error(AH_ERR_INVALID, "ah_download: bad argument");
    if (dtype == AH_F16) {
        std::vector<uint16_t> h((size_t)n);
        AH_HIP(hipMemcpyAsync(h.data(), dptr, (size_t)n * 2, hipMemcpyDeviceToHost, d->stream));
        AH_HIP(hipStreamSynchronize(d->stream));
        for (int64_t i = 0; i < n; i++) dst[i] = ah_f16_to_f32(h[i]);
    } else {
        AH_HIP(hipMemcpyAsync(dst, dptr, (size_t)n * 4, hipMemcpyDeviceToHost, d->stream));
        AH_HIP(hipStreamSynchronize(d->stream));
    }
    return AH_OK;
}

int ah_upload_bytes(ah_device *d, void *dptr, const void *src, int64_t nbytes) {
    if (!d || !dptr || (!src && nbytes)) return set_error(AH_ERR_INVALID, "ah_upload_bytes: bad argument");
    AH_HIP(hipMemcpyAsync(dptr, src, (size_t)nbytes, hipMemcpyHostToDevice, d->stream));
    AH_HIP(hipStreamSynchronize(d->stream));
    return AH_OK;
}

int ah_download_bytes(ah_device *d, void *dst, const void *dptr, int64_t nbytes) {
    if (!d || !dptr || (!dst && nbytes)) return set_error(AH_ERR_INVALID, "ah_download_bytes: bad argument");
    AH_HIP(hipMemcpyAsync(dst, dptr, (size_t)nbytes, hipMemcpyDeviceToHost, d->stream));
    AH_HIP(hipStreamSynchronize(d->stream));
    return AH_OK;
}

// ── modules ─────────────────────────────────────────────────────────────────

int ah_module_get(ah_device *d, const char *source, const char *entry, ah_kernel **out) {
    if (!d || !source || !out) return set_error(AH_ERR_INVALID, "ah_module_get: null argument");
    std::string ename = entry ? entry : "kernel";
    std::string key = ename + '\x1f' + source;
    auto it = d->modules.find(key);
    if (it != d->modules.end()) {
        *out = it->second;
        return AH_OK;
    }
    ah_kernel *k = new ah_kernel();
    // A WGSL kernel that is a plain contraction runs the hand-written MFMA template instead of its
    // rendering (wgsl_match.cpp); AH_WGSL_TEMPLATES=0 turns the selection off.
    std::string matched;
    const char *sel = getenv("AH_WGSL_TEMPLATES");
    const bool select = !(sel && strcmp(sel, "0") == 0);
    if (select && strstr(source, "@compute") && wgsl_match_contraction(source, &matched)) {
        int rc = template_create(matched.c_str(), &k->tmpl);
        if (rc != AH_OK) { delete k; return rc; }
    } else if (strncmp(source, "tmpl:", 5) == 0) {
        int rc = template_create(source, &k->tmpl);
        if (rc != AH_OK) { delete k; return rc; }
    } else {
        // The reference's schedule cache delivers kernels as rendered WGSL (schedule/cache.go:69-100):
        // such a source is first rendered as HIP by the WGSL-subset translator (wgsl.cpp).
        std::string hip_src = source;
        const bool from_wgsl = strstr(source, "@compute") != nullptr;
        if (from_wgsl) {
            std::string err;
            const char *wv = getenv("AH_WGSL_WAVE");   // "0": one thread per output, as the WGSL is written
            const bool try_wave = !(wv && strcmp(wv, "0") == 0);
            hip_src = wgsl_to_hip(source, &err, try_wave ? &k->wave : nullptr);
            if (hip_src.empty()) {
                delete k;
                return set_error(AH_ERR_COMPILE, "wgsl: %s", err.c_str());
            }
        }
        hiprtcProgram prog;
        if (hiprtcCreateProgram(&prog, hip_src.c_str(), "anneal_kernel.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
            delete k;
            return set_error(AH_ERR_COMPILE, "hiprtcCreateProgram failed");
        }
        std::string arch = "--offload-arch=" + d->arch.substr(0, d->arch.find(':'));
        // No packed FP32 VALU ops in generated code either (same flag as the library build); WGSL
        // kernels are compiled without FMA contraction (each WGSL operation rounds on its own) and
        // with wrapping signed arithmetic (WGSL i32 overflow wraps).
        const char *opts[] = {arch.c_str(), "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                              "-packed-fp32-ops", "-ffp-contract=off", "-fwrapv"};
        hiprtcResult rc = hiprtcCompileProgram(prog, from_wgsl ? 9 : 7, opts);
        if (rc != HIPRTC_SUCCESS) {
            size_t ls = 0;
            hiprtcGetProgramLogSize(prog, &ls);
            std::string log(ls, '\0');
            if (ls) hiprtcGetProgramLog(prog, &log[0]);
            hiprtcDestroyProgram(&prog);
            delete k;
            return set_error(AH_ERR_COMPILE, "hiprtc: %s", log.c_str());
        }
        size_t cs = 0;
        hiprtcGetCodeSize(prog, &cs);
        std::vector<char> code(cs);
        hiprtcGetCode(prog, code.data());
        hiprtcDestroyProgram(&prog);
        hipError_t e = hipModuleLoadData(&k->module, code.data());
        if (e == hipSuccess) e = hipModuleGetFunction(&k->function, k->module, ename.c_str());
        if (e != hipSuccess) {
            if (k->module) hipModuleUnload(k->module);
            delete k;
            return fail_hip(e, "hipModuleLoadData/GetFunction");
        }
    }
    d->modules[key] = k;
    *out = k;
    return AH_OK;
}

int ah_launch(ah_device *d, ah_kernel *k, const uint32_t grid[3], const uint32_t block[3], void *const *ptrs,
              int32_t n_ptrs, const int32_t *scalars, int32_t n_scalars) {
    if (!d || !k) return set_error(AH_ERR_INVALID, "ah_launch: null argument");
    if (k->tmpl) return k->tmpl->run(d, k->tmpl, ptrs, n_ptrs, scalars, n_scalars);
    if (!grid || !block) return set_error(AH_ERR_INVALID, "ah_launch: null grid/block");
    uint32_t g[3] = {grid[0], grid[1], grid[2]}, b[3] = {block[0], block[1], block[2]};
    if (k->wave) {   // one 64-lane block per original thread
        for (int a = 0; a < 3; a++) { g[a] = grid[a] * block[a]; b[a] = 1; }
        b[0] = 64;
    }
    std::vector<void *> args;
    std::vector<void *> pv(ptrs, ptrs + n_ptrs);
    std::vector<int32_t> sv(scalars, scalars + n_scalars);
    for (auto &p : pv) args.push_back(&p);
    for (auto &s : sv) args.push_back(&s);
    AH_HIP(hipModuleLaunchKernel(k->function, g[0], g[1], g[2], b[0], b[1], b[2], 0, d->stream, args.data(), nullptr));
    return AH_OK;
}

// ── timing ──────────────────────────────────────────────────────────────────

int ah_timer_start(ah_device *d) {
    if (!d) return set_error(AH_ERR_INVALID, "ah_timer_start: null device");
    if (!d->t0) {
        AH_HIP(hipEventCreateWithFlags(&d->t0, hipEventDisableSystemFence));   // timing only
        AH_HIP(hipEventCreateWithFlags(&d->t1, hipEventDisableSystemFence));
    }
    AH_HIP(hipEventRecord(d->t0, d->stream));
    return AH_OK;
}

int ah_timer_stop(ah_device *d, double *ms) {
    if (!d || !ms || !d->t0) return set_error(AH_ERR_INVALID, "ah_timer_stop: timer not started");
    AH_HIP(hipEventRecord(d->t1, d->stream));
    AH_HIP(hipEventSynchronize(d->t1));
    float f = 0.0f;
    AH_HIP(hipEventElapsedTime(&f, d->t0, d->t1));
    *ms = f;
    return AH_OK;
}

// ── graphs ──────────────────────────────────────────────────────────────────

int ah_graph_begin(ah_device *d) {
    if (!d) return set_error(AH_ERR_INVALID, "ah_graph_begin: null device");
    AH_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeRelaxed));
    return AH_OK;
}

int ah_graph_end(ah_device *d, ah_graph **out) {
    if (!d || !out) return set_error(AH_ERR_INVALID, "ah_graph_end: null argument");
    ah_graph *g = new ah_graph();
    hipError_t e = hipStreamEndCapture(d->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g->graph) hipGraphDestroy(g->graph);
        delete g;
        return fail_hip(e, "graph capture");
    }
    *out = g;
    return AH_OK;
}

int ah_graph_replay(ah_device *d, ah_graph *g) {
    if (!d || !g) return set_error(AH_ERR_INVALID, "ah_graph_replay: null argument");
    AH_HIP(hipGraphLaunch(g->exec, d->stream));
    return AH_OK;
}

void ah_graph_destroy(ah_graph *g) {
    if (!g) return;
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
}

}  // extern "C"

extern "C" int ah_wgsl_template_key(const char *wgsl, char *buf, int32_t cap) {
    if (!wgsl || !buf || cap <= 0) return set_error(AH_ERR_INVALID, "ah_wgsl_template_key: null argument");
    std::string key;
    if (!ah::wgsl_match_contraction(wgsl, &key)) {
        buf[0] = 0;
        return AH_OK;
    }
    snprintf(buf, (size_t)cap, "%s", key.c_str());
    return AH_OK;
}

extern "C" int ah_wgsl_plan(const char *wgsl, char *buf, int32_t cap) {
    if (!wgsl || !buf || cap <= 0) return set_error(AH_ERR_INVALID, "ah_wgsl_plan: null argument");
    std::string out;
    const char *sel = getenv("AH_WGSL_TEMPLATES");
    if (!(sel && strcmp(sel, "0") == 0) && ah::wgsl_match_contraction(wgsl, &out)) {
    } else {
        std::string err;
        bool wave = false;
        const char *wv = getenv("AH_WGSL_WAVE");
        const bool try_wave = !(wv && strcmp(wv, "0") == 0);
        if (ah::wgsl_to_hip(wgsl, &err, try_wave ? &wave : nullptr).empty()) return set_error(AH_ERR_COMPILE, "wgsl: %s", err.c_str());
        out = wave ? "wave" : "thread";
    }
    snprintf(buf, (size_t)cap, "%s", out.c_str());
    return AH_OK;
}
