/*
 * anneal_hip.h — C ABI of libanneal_hip.so, the MI355X (gfx950) backend for anneal's training hot path.
 *
 * Plain C types only (pointers, sizes, int codes). Every call returns AH_OK (0) or an AH_ERR_* code;
 * the message of the last failure on the calling thread is available from ah_last_error().
 * A device handle serializes all work onto one HIP stream; calls on one handle are not re-entrant
 * (the reference funnels every call onto a single owner thread: backend/webgpu/open.go:68-80).
 *
 * Each declaration names the reference interface it replaces (paths inside georgebuilds/anneal).
 */
#ifndef ANNEAL_HIP_H
#define ANNEAL_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AH_OK 0
#define AH_ERR_INVALID 1     /* bad argument / shape / handle */
#define AH_ERR_HIP 2         /* HIP runtime error */
#define AH_ERR_UNSUPPORTED 3 /* dtype or feature the device lacks (fail closed, executor.go:42-50) */
#define AH_ERR_COMPILE 4     /* hiprtc compilation failed */
#define AH_ERR_NOMEM 5

/* Buffer element types; numbering follows the reference's dtype set used on the device boundary
 * (backend/webgpu/executor.go:470-528): f16 is 2 bytes, every other type travels in 4 bytes. */
enum { AH_F32 = 0, AH_F16 = 1, AH_BF16 = 2, AH_I32 = 3, AH_BOOL = 4, AH_U32 = 5 };

typedef struct ah_device ah_device;
typedef struct ah_kernel ah_kernel;
typedef struct ah_graph ah_graph;
typedef struct ah_trainer ah_trainer;
typedef struct ah_plan ah_plan;

typedef struct {
    int32_t has_f16;     /* shader-f16 equivalent (always 1 on gfx950) */
    int32_t has_bf16;
    int32_t cu_count;
    int32_t wavefront;   /* 64 */
    int64_t hbm_bytes;
    int64_t lds_bytes_per_block;
    char arch[64];       /* e.g. "gfx950:sramecc+:xnack-" */
} ah_caps;

/* ── 1. device ───────────────────────────────────────────────────────────────
 * Replaces webgpu.Open (backend/webgpu/open.go:89) and Executor.Close (backend/device.go:12). */
const char *ah_last_error(void);
int ah_open(int ordinal, ah_device **out);
void ah_close(ah_device *dev);
int ah_get_caps(ah_device *dev, ah_caps *out);
int ah_sync(ah_device *dev);

/* ── 2. buffers and the dtype codec ──────────────────────────────────────────
 * Replaces the per-Run CreateBuffer / WriteBuffer / readBuffer of backend/webgpu/executor.go:83-179,397-468
 * and the codec of executor.go:470-528 / uop/dtype.go:392-487 (f32->f16 round-to-nearest-even with the
 * reference's NaN and overflow rules; bf16 = top 16 bits carried in a 4-byte slot). */
int ah_buf_alloc(ah_device *dev, int64_t n_elems, int32_t dtype, void **dptr);
int ah_buf_free(ah_device *dev, void *dptr);
int ah_upload(ah_device *dev, void *dptr, const float *src, int64_t n, int32_t dtype);
int ah_download(ah_device *dev, float *dst, const void *dptr, int64_t n, int32_t dtype);
int ah_upload_bytes(ah_device *dev, void *dptr, const void *src, int64_t nbytes);
int ah_download_bytes(ah_device *dev, void *dst, const void *dptr, int64_t nbytes);
uint16_t ah_f32_to_f16(float f);   /* uop/dtype.go:392 Float32ToFloat16 */
float ah_f16_to_f32(uint16_t h);   /* uop/dtype.go:447 Float16ToFloat32 */

/* ── 3./4. modules and launches ──────────────────────────────────────────────
 * Replaces CreateShaderModule + pipeline creation + Dispatch (backend/webgpu/executor.go:254-395).
 * `source` is either HIP C++ source (compiled once by hiprtc for gfx950, cached by source hash) or a
 * template key "tmpl:<name>;k=v;..." selecting a hand-written kernel (the names and their keys are
 * listed in anneal_amd/csrc/templates.cpp).
 * Kernel arguments: n_ptrs device pointers (data0 = output, data1.. = inputs, PARAM order as in
 * codegen/wgsl.go:58-76), then n_scalars int32 values (the params_n uniform of symbolic kernels). */
int ah_module_get(ah_device *dev, const char *source, const char *entry, ah_kernel **out);

/* The WGSL anneal's codegen renders (codegen/wgsl.go:41-238 RenderWGSL, the string the schedule cache
 * keeps in ExecItem.WGSL, schedule/cache.go:69-100) is also accepted as `source` by ah_module_get / ah_run:
 * it is rendered as HIP C++ (entry point `kernel`, the storage bindings in binding order, then the four
 * int32 fields of params_n for symbolic kernels) and compiled by hiprtc. This call exposes that rendering
 * on its own (no device needed): writes at most cap bytes of NUL-terminated HIP source to out and the
 * full size to *needed; AH_ERR_COMPILE if the WGSL is outside the subset the reference emits. */
int ah_translate_wgsl(const char *wgsl, char *out, int64_t cap, int64_t *needed);
/* Template selection for a rendered WGSL kernel (host only, no device). The kernel's body, in the form
 * codegen/lower.go:98-719 lowers and codegen/wgsl.go:41-386 renders it (one let per ALU node and load,
 * GIDVar axes, one accumulator and loop per reduce, f16 reduces widened and narrowed with f16(acc),
 * params_n for a symbolic batch), is parsed with every let substituted, and two families select a
 * hand-written kernel: a contraction REDUCE(ADD, MUL(a, b)) whose operands are loads, ReLU prologues
 * max(x, 0.0) or ReLU-backward mask prologues select(0.0, adj, z == max(z, 0.0)), stored as acc,
 * f16(acc), c*acc, acc + bias[n] or max(acc + bias[n], 0.0) -> "tmpl:gemm;..." (dtype f32 or f16, M/N/K
 * "sym" where symbolic); and a reduction REDUCE(ADD|MAX, load) along a row or down a column (or over a
 * whole 1-D buffer) stored into f32 -> "tmpl:reduce;...". Index expressions must evaluate as affine with
 * zero offset over the axes. Writes the key ah_module_get runs in the kernel's place to buf, or "". No
 * counterpart in the reference, whose backend renders every kernel: it exposes the selection
 * ah_module_get and ah_run make (AH_WGSL_TEMPLATES=0 turns it off). */
int ah_wgsl_template_key(const char *wgsl, char *buf, int32_t cap);
/* How ah_module_get runs a rendered WGSL kernel (host only): writes the template key when one is selected
 * (as above), "wave" when the kernel is rendered in the wave-per-output form (a single-reduce kernel:
 * one 64-lane wave per output element, the lanes striding the outermost reduce loop and combining their
 * partials with a shuffle tree, AH_WGSL_WAVE=0 turns it off), or "thread" for the one-thread-per-output
 * rendering of ah_translate_wgsl. AH_ERR_COMPILE if the WGSL is outside the subset. */
int ah_wgsl_plan(const char *wgsl, char *buf, int32_t cap);
int ah_launch(ah_device *dev, ah_kernel *k, const uint32_t grid[3], const uint32_t block[3],
              void *const *ptrs, int32_t n_ptrs, const int32_t *scalars, int32_t n_scalars);

/* ── 5. timing ───────────────────────────────────────────────────────────────
 * Replaces Benchmarker.Benchmark's wall-clock loop (backend/webgpu/benchmark.go:18-208) with hipEvents. */
typedef struct {
    double min_us, median_us, max_us, mean_us, stddev_us, cv;   /* backend/device.go:16-24 */
} ah_bench_result;

/* Wall time of everything enqueued on the device stream between start and stop (hipEvents). */
int ah_timer_start(ah_device *dev);
int ah_timer_stop(ah_device *dev, double *ms);

/* ── 6. graphs (JIT replay) ──────────────────────────────────────────────────
 * Replaces tensor.JIT's replay of captured ExecItems (tensor/jit.go:178-215): everything enqueued on the
 * device stream between begin and end is captured and can be replayed without host scheduling. */
int ah_graph_begin(ah_device *dev);
int ah_graph_end(ah_device *dev, ah_graph **out);
int ah_graph_replay(ah_device *dev, ah_graph *g);
void ah_graph_destroy(ah_graph *g);

/* ── Executor mirror (backend.Executor / Benchmarker / SymbolicExecutor, backend/device.go:10-37) ──
 * Items follow schedule.ExecItem (schedule/exec.go:6-32): bufs[0] is the output, bufs[1..] inputs in
 * PARAM order; slot >= 0 marks a slot shared by non-overlapping lifetimes, -1 a leaf or final output.
 * Final outputs are the bufs[0] that no later item reads; they are returned widened to f32 (4-byte
 * integer types as raw bits), keyed by uop_idx, in ah_output arrays owned by the library. */
typedef struct {
    uint32_t uop_idx;
    int64_t size;        /* elements; 0 when the leading dim is symbolic */
    int32_t dtype;
    int32_t slot;
    int32_t rank;
    const int64_t *shape;
} ah_buffer_desc;

typedef struct {
    const char *source;           /* HIP source or "tmpl:" key (replaces the WGSL string field) */
    const ah_buffer_desc *bufs;
    int32_t n_bufs;
    const char *const *sym_vars;
    int32_t n_sym_vars;
    int32_t local_size[3];
    int32_t workgroup_count[3];
} ah_exec_item;

typedef struct {
    uint32_t uop_idx;
    const float *data;
    int64_t n;
} ah_input;

typedef struct {
    uint32_t uop_idx;
    float *data;
    int64_t n;
} ah_output;

int ah_run(ah_device *dev, const ah_exec_item *items, int32_t n_items, const ah_input *inputs, int32_t n_inputs,
           ah_output **outputs, int32_t *n_outputs);                       /* Executor.Run, device.go:11 */
int ah_run_symbolic(ah_device *dev, const ah_exec_item *items, int32_t n_items, const ah_input *inputs,
                    int32_t n_inputs, const char *const *bind_names, const int64_t *bind_values,
                    int32_t n_bind, ah_output **outputs, int32_t *n_outputs); /* RunSymbolic, device.go:35-37 */
int ah_benchmark(ah_device *dev, const ah_exec_item *item, int32_t warmup, int32_t iterations,
                 ah_bench_result *out);                                     /* Benchmark, device.go:27-29 */
void ah_outputs_free(ah_output *outputs, int32_t n);

/* Persistent plans: the device half of tensor.JIT (tensor/jit.go:47-359), which captures one item list and
 * replays it through Run / RunSymbolic with fresh leaf data every step (replayStatic / replaySym,
 * jit.go:178-215). ah_plan_create copies the items, resolves every kernel once (compile errors surface here)
 * and ah_plan_run runs them with Run's contract (zeroed buffers, leaves from `inputs`, final outputs
 * returned as by ah_run). Buffers stay allocated between runs and grow when a larger symbolic binding
 * arrives. With AH_PLAN_GRAPH the kernel sequence of each binding is captured once as a HIP graph and
 * replayed afterwards (uploads and downloads stay outside the graph). ah_plan_stats reports
 * (captures, replays) like JIT.JITStats (jit.go:71-74). A plan belongs to its device handle's stream. */
#define AH_PLAN_GRAPH 1
int ah_plan_create(ah_device *dev, const ah_exec_item *items, int32_t n_items, ah_plan **out);
int ah_plan_run(ah_plan *plan, const ah_input *inputs, int32_t n_inputs, const char *const *bind_names,
                const int64_t *bind_values, int32_t n_bind, int32_t flags, ah_output **outputs, int32_t *n_outputs);
int ah_plan_stats(const ah_plan *plan, int64_t *captures, int64_t *replays);
void ah_plan_destroy(ah_plan *plan);

/* ── Hot-path kernels, callable directly ────────────────────────────────────── */

/* GEMM-shaped REDUCE(ADD, MUL) with fused epilogue (tensor/reduce.go:105-166 as scheduled for
 * Linear.Forward nn.go:154-162 and the backward rules gradient_ruleset.go:137-140,207-233,285-306).
 * C[m,n] = epi(sum_k A(m,k) B(n,k)); A stored [M,K] (ta=0) or [K,M] (ta=1); B [N,K] (tb=0) or [K,N] (tb=1). */
enum { AH_EPI_STORE = 0, AH_EPI_BIAS = 1, AH_EPI_BIAS_RELU = 2, AH_EPI_MSE = 3, AH_EPI_MASK = 4, AH_EPI_SGD = 5 };
typedef struct {
    int32_t dtype;          /* AH_F32 or AH_F16 (operands); accumulation is always f32 */
    int32_t epi;
    int32_t ta, tb;
    int32_t M, N, K;
    const void *A;
    const void *B;
    int64_t lda, ldb;
    void *C;
    int64_t ldc;
    const void *bias;
    const void *aux;
    int64_t ldaux;
    float scale;
    float *colsum;
    float *W32;
    void *W16;
    float lr;
    float *gout;
    float *lossacc;
    int32_t tile;           /* 0 = auto, 64, 128, 256 (register-staged f32 kernel), 1000 + i (f32 direct-to-LDS
                               configuration i, 0..4; see ah_gemm_tune) */
    int32_t variant;        /* f16 kernel variant: 0 = auto (the tuned choice if any), 1..39 = fixed tile /
                               wave / fetch / k-group / MFMA-shape choices (table Var<V>, gemm16_kernel.h);
                               the knob a BEAM-style search times (codegen/beam.go:41-541) */
} ah_gemm_desc;
int ah_gemm(ah_device *dev, const ah_gemm_desc *d);

/* BEAM over the f16 kernel variants (replaces BeamSearch timing candidate Opt sequences per kernel and
 * caching the winner, codegen/beam.go:41-541, :118-169). Times every variant of the contraction d
 * describes (iterations launches each, after one warm-up, on the device stream with hipEvents; two passes,
 * each variant timed by the lower of its two means), returns
 * the fastest and its mean time, and caches the choice on the device: later launches of the same
 * (ta, tb, M, N, K) with variant 0 use it. d is launched as given, so its outputs must be scratch
 * (the epilogue runs 2 * (iterations + 1) times per variant). Variants without k-groups differ only in
 * tiling and scheduling and accumulate each output over k in the same order (bit-identical results);
 * the k-group variants 10, 11, 15, 25, 28, 31 and 35-38 add two k-halves, which rounds differently in f32 (relative
 * 1e-6 level). For an f32 contraction (dtype AH_F32) the candidates are the f32 kernel's (tile, k-groups,
 * splits of K across workgroups) configurations and the direct-to-LDS kernel's, 58 in all, and
 * *best_variant is the winner's index: 0 is the shape's automatic choice, then the register-staged
 * kernel's tile 64 and 128 each with k-groups auto / 1 / 2 / 4 (as the tile admits) and splits auto / 1 /
 * 2 / 4 / 8 / 16 in that nesting order (a fixed k-group count takes no automatic split, so splits auto is
 * listed only with k-groups auto), indices 1-37; then the direct-to-LDS configurations 0-4 (tile 64 with
 * k 64 x 3 stages, 64 x 4, 32 x 4; tile 128 with k 32 x 4, 64 x 2), indices 38-42, then each of those
 * with K split across 2 / 4 / 8 workgroups (43-57; the partials folded in split order as the
 * register-staged kernel folds them). The automatic choice is
 * the direct-to-LDS kernel on 64-wide tiles when they number at least 256 (at least 128 for K <= 1024),
 * the register-staged kernel otherwise. Later f32 launches of the shape with tile, k-groups and splits all automatic use the
 * winner. Configurations add K in different orders, so their results differ at the rounding level;
 * those of one tile width without k-groups or splits give the same bits in either kernel. */
int ah_gemm_tune(ah_device *dev, const ah_gemm_desc *d, int32_t iterations, int32_t *best_variant, double *best_us);
/* BEAM's disk cache (codegen/beam.go:118-169): save (save != 0) the device's tuned choices to path, one
 * "dtype/ta/tb/M/N/K variant" line each under a header naming the gfx arch, or merge a saved file into
 * the device's cache (a file timed on another arch is ignored). The config-3 trainer loads and rewrites
 * the file named by the environment variable AH_GEMM_TUNE_CACHE around its tuning. */
int ah_gemm_tune_cache(ah_device *dev, const char *path, int32_t save);

/* ── The Opt seam and BEAM over the HIP templates ─────────────────────────────
 * Replaces codegen/opt.go's ApplyOpt/ApplyOpts (:29-72, :559-567) and codegen/beam.go's ActionSpace,
 * BeamSearch, BeamApplyToItems and disk cache (:41-541). An Opt {kind, axis, arg} (opt.go:41-46) edits a
 * template key's tuning parameters instead of an AST: LOCAL(axis 0|1, 8|16|32) the waves along M or N
 * (arg/8), UPCAST(axis 0|1, 2|4) the MFMA register tile per wave (f32 kernel: tile 64*arg), TILE(axis 2,
 * 8|16|32) the LDS stage (k 32 x 4 stages, 64 x 2, 64 x 3), VECTORIZE(axis 2, 4) 16-byte asm LDS-DMA
 * staging (f32: the direct-to-LDS kernel, whose stage TILE then sets; the key gets dma=i);
 * GROUP(axis 2, 2|4) k-groups, SCHEDULE(axis 0, 5..7) the DMA/fragment-read interleave and MFMA(axis 2,
 * 16|32) the f16 kernel's MFMA shape (16x16x32 or 32x32x16; bit-identical results) are MI355X additions.
 * Only "tmpl:gemm" keys have tunable parameters. */
enum { AH_OPT_IDENTITY = 0, AH_OPT_LOCAL = 1, AH_OPT_TILE = 2, AH_OPT_UPCAST = 3, AH_OPT_VECTORIZE = 4,
       AH_OPT_GROUP = 5, AH_OPT_SCHEDULE = 6, AH_OPT_MFMA = 7 };
typedef struct {
    int32_t kind, axis, arg;
} ah_opt;
/* ApplyOpts: the key with the sequence applied (NUL-terminated, at most cap bytes; *needed = full size);
 * AH_ERR_UNSUPPORTED if an Opt does not apply or the result is not an instantiated kernel. */
int ah_apply_opts(const char *key, const ah_opt *opts, int32_t n, char *out, int64_t cap, int64_t *needed);
/* ActionSpace (beam.go:53-72): every single Opt that changes the key's kernel; *n = count, at most cap
 * written to out. */
int ah_action_space(const char *key, ah_opt *out, int32_t cap, int32_t *n);
typedef struct {
    double min_us, base_us;   /* winner's and the unmodified kernel's min-of-N times */
    int32_t searched;         /* candidates benchmarked */
    int32_t from_cache;
    int32_t n_opts;
    ah_opt opts[8];           /* the winning sequence (empty: identity) */
} ah_beam_result;
/* BeamSearch (beam.go:271-408) over item (a "tmpl:" item, buffers as for ah_benchmark): beam width and
 * depth, each candidate timed by ah_benchmark (warmup, iters; min), kept only if its output is
 * bit-identical to the unmodified kernel's on fixed inputs (beam.go:410-451). The winner is cached per
 * process keyed by the FNV-64a hash of the item's key; a cached kernel is re-timed, not searched. */
int ah_beam_search(ah_device *dev, const ah_exec_item *item, int32_t width, int32_t depth, int32_t warmup,
                   int32_t iters, ah_beam_result *out);
/* BeamApplyToItems' cache hit (beam.go:470-541): the cached specialised key for key, or key itself; the
 * stored hash of the specialised key guards against key-hash collisions. */
int ah_beam_apply(const char *key, char *out, int64_t cap, int64_t *needed);
/* The persistent cache (beam.go:100-150): save (save != 0) every cached winner to path, or merge path
 * into the process cache. */
int ah_beam_cache(const char *path, int32_t save);
void ah_beam_reset(void);   /* BeamCacheReset (beam.go:213) */

/* Softmax cross-entropy forward+backward composed from reference ops (one wave64 per row):
 * m=Max, zs=z-m, e=Exp(zs), s=Sum e, logp=zs-Log(s), loss=Sum(onehot*logp)*(-1/B); dz includes the
 * row-max path with its tie split (tensor/gradient_ruleset.go:307-320). */
int ah_softmax_ce(ah_device *dev, const float *z, const int32_t *labels, int32_t B, int32_t C, float *dz,
                  float *loss);

/* Config-5 chain: Y = Shrink(Pad(Permute(X,(1,0)))), S = softmax(Y, 1),
 * out = S * recip(sqrt(mean(S*S,1) + 1e-6)) * g; loss = Sum(out); returns dX [R,Cc], dg [Cc]. */
int ah_chain_step(ah_device *dev, const float *X, const float *g, int32_t R, int32_t Cc, float *dX, float *dg,
                  float *loss);
/* ah_chain_step without allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops). The chain's workspace is a
 * file-scope device array of 2^22 floats (16 MiB per GPU, held until the process ends), so
 * 64 + max(ceil(R/64)*Cc*4 + Cc*8 + ceil(Cc/16), Cc/16) must not exceed 2^22 (config 5, 8192 x 4096, needs 2.13M);
 * larger shapes fail with AH_ERR_INVALID. Asynchronous: the chain kernels (one at R = 8192, else three) are enqueued on the device
 * stream and the call returns (ah_sync waits). Every call on one GPU shares that GPU's workspace, so
 * calls that overlap on one GPU (several device handles or host threads) race. */
int ah_chain_step_noalloc(ah_device *dev, const float *X, const float *g, int32_t R, int32_t Cc, float *dX,
                          float *dg, float *loss);

/* ── Device-resident training steps (one BASELINE config each) ───────────────
 * Replaces the reference step pattern: graph build -> tensor.Backward -> one tensor.Realize per gradient
 * -> host SGD (examples/mlp.go:112-142, tensor/nn/nn.go:69-106). Parameters stay resident as f32 masters
 * (plus f16 copies for f16 configs); SGD runs on the device inside the backward kernels. */
enum {
    AH_TRAIN_MLP_CE = 1,    /* dims {Bmax, D, H, C}: configs 1 and 4 */
    AH_TRAIN_CONVNET = 2,   /* dims {N, Hin, C1, C2, NC}: config 2 */
    AH_TRAIN_MLP3_F16 = 3,  /* dims {B, D0, D1, D2, D3[, adjoint]}: config 3; adjoint 1 keeps the masked
                               adjoints dZ2, dZ1 at f32 precision as two f16 planes (hi, lo) and contracts
                               both (dH1, dW2, dW1 then cost two passes over K); 0 (default) rounds them
                               to f16 */
    AH_TRAIN_CHAIN = 4,     /* dims {R, Cc}: config 5 */
};
/* Slot numbering per kind (host arrays are f32 unless noted; labels are int32):
 *  MLP_CE : 0 x, 1 labels, 2 W1, 3 b1, 4 W2, 5 b2, 6 loss, 7 dW1, 8 db1, 9 dW2, 10 db2,
 *           11 H1 (the last step's ReLU outputs, batch rows first; -0.0 marks a dead unit) — read only
 *  CONVNET: 0 x, 1 labels, 2 cw1, 3 cb1, 4 cw2, 5 cb2, 6 fw, 7 fb, 8 loss, 9 dcw1, 10 dcb1, 11 dcw2,
 *           12 dcb2, 13 dfw, 14 dfb
 *  MLP3   : 0 x, 1 t, 2 W1, 3 b1, 4 W2, 5 b2, 6 W3, 7 b3, 8 loss, 9 dW1, 10 db1, 11 dW2, 12 db2,
 *           13 dW3, 14 db3, 15 loss_sum (the f32 sum of squares before the f16 narrowing of the loss),
 *           16 H1, 17 H2 (the f16 ReLU outputs of the last step, widened; -0.0 marks a dead unit),
 *           18 d = f16(P - t) (the last step's loss adjoint before the factor 2/(B*D3)) — read only
 *  CHAIN  : 0 X, 1 g, 2 loss, 3 dX, 4 dg
 * Gradient slots are filled only by steps run with AH_STEP_STORE_GRADS.
 * Creating an MLP3 trainer tunes its f16 contractions for shapes the device has not tuned yet: each alone
 * (ah_gemm_tune), then each variant again inside running steps on hash-filled buffers (≈1.9 s in all at the
 * config-3 shape); every parameter, data and accumulator buffer is zero when create returns. */
#define AH_STEP_STORE_GRADS 1
#define AH_STEP_GRAPH 2      /* capture the step once per batch size as a hipGraph and replay it (tensor.JIT) */
int ah_trainer_create(ah_device *dev, int32_t kind, const int64_t *dims, int32_t n_dims, float lr,
                      ah_trainer **out);
void ah_trainer_destroy(ah_trainer *t);
int ah_trainer_set(ah_trainer *t, int32_t slot, const void *host, int64_t n);
int ah_trainer_get(ah_trainer *t, int32_t slot, void *host, int64_t n);
int ah_trainer_step(ah_trainer *t, int64_t batch, int32_t flags);
/* n consecutive steps (tensor.JIT's replay loop, tensor/jit.go:176-215, with the inputs left in place).
 * With AH_STEP_GRAPH the steps run as hipGraph launches of up to 16 steps each, each graph captured once
 * per (batch, flags, steps) and replayed: a graph launch has a fixed host and GPU cost, paid once per
 * graph rather than once per step. Without it, n eager steps. */
int ah_trainer_steps(ah_trainer *t, int64_t batch, int32_t flags, int32_t n);
/* Per-kernel probe: hipEvents around the index-th kernel launch of every following step. */
int ah_trainer_probe(ah_trainer *t, int32_t kernel_index);
/* Probe of launches first..last of every following step: one hipEvent before launch `first`, one after
 * launch `last`; last = first - 1 records the two events back to back (their own cost alone). Two spans
 * that differ by one launch give that launch's share of the step with the events' cost cancelled. */
int ah_trainer_probe_span(ah_trainer *t, int32_t first, int32_t last);
int ah_trainer_probe_read(ah_trainer *t, double *total_ms, int64_t *count);
int ah_trainer_kernel_count(ah_trainer *t, int64_t batch, int32_t *count);
/* Name of the index-th launch of a step, as counted by the last ah_trainer_kernel_count (NUL-terminated,
 * truncated to cap bytes). The reference's Benchmark reports per-kernel results by kernel
 * (backend/webgpu/benchmark.go); this names the trainer's launches for the same purpose. */
int ah_trainer_kernel_name(ah_trainer *t, int32_t index, char *buf, int32_t cap);

/* ── Checkpoint formats (host side; no device needed) ─────────────────────────
 * Readers for safetensors (tensor/safetensors/safetensors.go:150-434 Load / LoadTensors), NumPy .npy and
 * .npz with stored or deflated members (tensor/npy/npy.go:41-466 Load / LoadNPZ), decoding every tensor to f32 with the reference's
 * dtype policy (safetensors.go:21-35, npy.go:3-16): F32 exact, F64 -> f32, F16 / BF16 widened (safetensors),
 * integers by value with an error past 2^24, BOOL -> 0/1, any other dtype an error naming it; Fortran-order
 * arrays come back in C order. The decoded values are what a trainer uploads with ah_trainer_set. */
typedef struct ah_ckpt ah_ckpt;
int ah_ckpt_open(const char *path, ah_ckpt **out);   /* format from the file's magic bytes */
int32_t ah_ckpt_count(const ah_ckpt *c);
int ah_ckpt_entry(const ah_ckpt *c, int32_t i, const char **name, const char **dtype, int32_t *rank,
                  const int64_t **shape, int64_t *n_elems);
int ah_ckpt_read(const ah_ckpt *c, int32_t i, float *out, int64_t n);
void ah_ckpt_close(ah_ckpt *c);
/* Writer for F32 safetensors checkpoints as safetensors.Save writes them (safetensors.go:75-146): names
 * sorted, header JSON {"name":{"dtype":"F32","shape":[..],"data_offsets":[a,b]},..} padded with spaces to
 * a multiple of 8 bytes, data little-endian in name order. */
int ah_safetensors_save(const char *path, int32_t n, const char *const *names, const float *const *data,
                        const int64_t *const *shapes, const int32_t *ranks);

#ifdef __cplusplus
}
#endif
#endif
