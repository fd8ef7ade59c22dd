// ah_internal.h — host-side internals shared by runtime.cpp, executor.cpp and plans.cpp.
#pragma once
#include <hip/hip_runtime.h>

#include <functional>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/anneal_hip.h"

namespace ah {

int set_error(int code, const char *fmt, ...);
int fail_hip(hipError_t e, const char *what);

#define AH_HIP(expr)                                   \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return ::ah::fail_hip(e_, #expr); \
    } while (0)

int64_t dtype_bytes(int32_t dtype);

// Built-in template kernel, selected by a "tmpl:" source key (templates.cpp). run() launches it on the
// device stream with the ExecItem's buffers (PARAM order) and the symbolic scalars.
struct TemplateKernel {
    std::string key, name;
    // PARAMs after data0 that the kernel writes (zero: the kernel accumulates into it, so it must start at 0)
    struct Side {
        int param;
        bool zero;
    };
    std::vector<Side> side;
    // bytes of device workspace the kernel needs for a symbolic binding (null: none); the workspace is the
    // template's own, grown by template_prepare (or on first use) and freed with the template
    std::function<int64_t(int64_t symval)> workspace;
    // bytes each PARAM must hold for a binding (entry j: PARAM j; 0: not read or written), from the key's
    // shape; the executor checks the bound buffers against it before anything is launched
    std::function<std::vector<int64_t>(int64_t symval)> bytes;
    void *ws = nullptr;
    int64_t ws_bytes = 0;
    std::function<int(ah_device *, TemplateKernel *self, void *const *ptrs, int32_t n_ptrs, const int32_t *scalars,
                      int32_t n_scalars)>
        run;
    ~TemplateKernel();
};

struct GemmDesc;
// A contraction launched with the device's tuned f16 variant when the descriptor leaves the choice open.
hipError_t gemm_dispatch(ah_device *dev, const GemmDesc &g);

}  // namespace ah

struct ah_kernel {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    // rendered in the wave-per-output form (wgsl.cpp): launched with one 64-lane block per thread of the
    // item's grid x block
    bool wave = false;
    ah::TemplateKernel *tmpl = nullptr;
};

struct ah_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    std::unordered_map<std::string, ah_kernel *> modules;
    std::string arch;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    // f16 GEMM variant chosen by ah_gemm_tune per (ta, tb, M, N, K); used when a launch asks for
    // variant 0 (the role of BEAM's cache, codegen/beam.go:118-169).
    std::unordered_map<std::string, int> gemm_variant;
    // This device's address of the chain's file-scope workspace (ah_chain_step_noalloc), set by ah_open.
    float *chain_scratch = nullptr;
    // Split-K workspace of the f32 tiled contractions (counters, then partial tiles), set up by ah_open.
    void *splitk_ws = nullptr;
};

struct ah_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace ah {
int template_create(const std::string &source, TemplateKernel **out);
// "tmpl:<name>;k=v;..." -> name and the k=v map.
std::unordered_map<std::string, std::string> template_key_params(const std::string &key, std::string *name);
// Grows the template's workspace for the binding symval (before a graph capture).
int template_prepare(TemplateKernel *t, int64_t symval);
std::string wgsl_to_hip(const std::string &src, std::string *err, bool *wave = nullptr);
// A "tmpl:gemm" key for a WGSL kernel that is a plain contraction (wgsl_match.cpp), else false.
bool wgsl_match_contraction(const std::string &src, std::string *key);
}
