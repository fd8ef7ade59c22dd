// templates.cpp — the "tmpl:" keys: hand-written gfx950 kernels an ExecItem can name instead of source.
//
// A key is "tmpl:<name>;k=v;...". Integer parameters may be "sym": they then take the bound value of the
// item's symbolic variable (the first int32 scalar of the launch, params_n in codegen/wgsl.go:58-76).
// Float parameters accept anything strtof reads, hex floats included (so 1/B can be given exactly).
// PARAM order follows the reference's item contract (schedule/exec.go:6-32): data0 is the output and
// data1.. the inputs. Some templates also write one or more later PARAMs ("side outputs": a loss partial,
// a per-row loss, a bias gradient); the executor treats those as produced by the item.
//
// Keys (shapes in elements, row-major):
//   gemm        data0 C [M,N], data1 A, data2 B (+ bias / aux / targets by epilogue). See template_gemm.
//   reduce      data0 out f32, data1 G [M,N] (dtype=f32|f16); op=sum|max|sumsq, axis=0 (out [N]) or 1
//               (out [M]), scale (applied to the sums); runs in f32 with a fixed order.
//   softmax_ce  data0 dz [B,C], data1 z [B,C], data2 labels i32 [B]; side data3 rowloss [B].
//               dz is the gradient of Sum(onehot*logp)*(-1/B); rowloss[b] = logp[b, label].
//   maxpool2d   data0 out [N,C,oH,oW], data1 x [N,C,H,W]; N,C,H,W,kh,kw,sh,sw.
//   maxpool2d_bwd  data0 dx [N,C,H,W], data1 x, data2 adj [N,C,oH,oW]; same parameters.
//   pool_relu_bwd  data0 dz [N,C,H,H], data1 dp [N,C,H/2,H/2], data2 h (tagged ReLU output), data3 p
//               (pooled h): 2x2 stride-2 pool backward with the tie split, then the ReLU mask.
//   conv2d      data0 y [N,Co,H,H], data1 x [N,Ci,H,H], data2 w [Co,Ci,3,3], data3 b [Co]; relu=0|1.
//   conv2d_relu_pool  data0 p [N,Co,H/2,H/2], data1 x, data2 w, data3 b; side data4 h [N,Co,H,H].
//   conv2d_bwd_x  data0 dx [N,Ci,H,H], data1 g [N,Co,H,H], data2 w.
//   conv2d_bwd_w  data0 dw [Co,Ci,3,3], data1 x [N,Ci,H,H], data2 g [N,Co,H,H].
//   conv2d_bwd_b  data0 db [Co], data1 g [N,Co,H,H].
//   sgd         data0 p' [n], data1 p, data2 g; p' = p - lr*(scale*g)  (Parameter.SGDStep, nn.go:69-76).
//   mse_loss    data0 loss [1], data1 per-wave partials [parts]; loss = f16(sum) * scale.
//   chain       data0 dX [R,Cc], data1 X [R,Cc], data2 g [Cc]; side data3 dg [Cc], data4 loss [1].
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>

#include "ah_internal.h"
#include "conv.h"
#include "gemm.h"
#include "itemops.h"
#include "rowops.h"

namespace ah {

// "tmpl:<name>;k=v;..." -> name and the k=v map.
std::unordered_map<std::string, std::string> template_key_params(const std::string &s, std::string *name) {
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

namespace {

constexpr int kEpiGrad = 100;   // key-only epilogue: SGD on a zeroed array (see template_gemm)


// Parsed parameters of one key; integers may be "sym" (resolved per launch).
struct Params {
    std::unordered_map<std::string, std::string> kv;
    std::string name;
    bool has(const char *k) const { return kv.count(k) != 0; }
    std::string str(const char *k, const char *dflt) const {
        auto it = kv.find(k);
        return it == kv.end() ? dflt : it->second;
    }
    bool sym(const char *k) const {
        auto it = kv.find(k);
        return it != kv.end() && it->second == "sym";
    }
    // -1 when absent; -2 when not an integer
    long integer(const char *k, long dflt = -1) const {
        auto it = kv.find(k);
        if (it == kv.end()) return dflt;
        char *end = nullptr;
        long v = strtol(it->second.c_str(), &end, 10);
        return (end && *end == 0 && !it->second.empty()) ? v : -2;
    }
    float real(const char *k, float dflt) const {
        auto it = kv.find(k);
        return it == kv.end() ? dflt : strtof(it->second.c_str(), nullptr);
    }
};

// An integer parameter that is either fixed or "sym".
struct Dim {
    long v = -1;
    bool sym = false;
    long at(const int32_t *sc, int32_t ns) const { return sym ? (ns > 0 ? sc[0] : -1) : v; }
    int64_t with(int64_t symv) const { return sym ? symv : v; }
};

int get_dim(const Params &p, const char *k, Dim *d, bool allow_sym, bool required = true, long dflt = -1) {
    if (p.sym(k)) {
        if (!allow_sym) return set_error(AH_ERR_INVALID, "tmpl %s: %s cannot be symbolic", p.name.c_str(), k);
        d->sym = true;
        return AH_OK;
    }
    long v = p.integer(k, dflt);
    if (v == -2 || (required && v < 0)) return set_error(AH_ERR_INVALID, "tmpl %s: %s required (integer)", p.name.c_str(), k);
    d->v = v;
    return AH_OK;
}

#define GET(k, d, sym) \
    do { int rc_ = get_dim(P, k, &d, sym); if (rc_) return rc_; } while (0)

// Resolves symbolic dims at launch; fails when a symbolic dim has no binding or a dim is negative.
#define AT(d, out)                                                                                     \
    long out = (d).at(sc, ns);                                                                         \
    if (out < 0) return set_error(AH_ERR_INVALID, "tmpl %s: symbolic dimension without a binding", key.c_str());

int need(const char *key, int32_t n_ptrs, int want) {
    if (n_ptrs < want) return set_error(AH_ERR_INVALID, "tmpl %s: needs %d buffers, got %d", key, want, n_ptrs);
    return AH_OK;
}

// Grows the template's own device workspace (kept for the device's lifetime; never under capture when
// the caller prepares items first, as ah_plan does). A new workspace starts zeroed.
int ensure_ws(TemplateKernel *t, int64_t bytes) {
    if (bytes <= t->ws_bytes) return AH_OK;
    if (t->ws) AH_HIP(hipFree(t->ws));
    t->ws = nullptr;
    t->ws_bytes = 0;
    AH_HIP(hipMalloc(&t->ws, (size_t)bytes));
    t->ws_bytes = bytes;
    AH_HIP(hipMemset(t->ws, 0, (size_t)bytes));
    return AH_OK;
}

// ── gemm ─────────────────────────────────────────────────────────────────────────────────────────
// "tmpl:gemm;dtype=f16|f32;epi=...;ta=0|1;tb=0|1;M=..;N=..;K=..[;scale=s][;lr=l][;variant=v][;tile=t;kg=g]
//  [;splits=s][;dma=i][;swap_ab=1][;wa=1][;wb=1][;wza=1][;wzb=1][;in_a=i;in_b=j;in_bias=k][;pa=relu|mask;za=z][;pb=relu|mask;zb=z]"
// swap_ab: A is the second input PARAM and B the first; in_a / in_b / in_bias name the PARAM of each role
// outright (a rendered kernel binds its inputs in the scheduler's order). Operand prologues, the
// elementwise ops the reference's scheduler inlines into a contraction's loop: pa=relu reads max(A, 0)
// (ReLU = Maximum(x, 0), tensor/nn/nn.go:111-114), pa=mask reads Where(Z == max(Z, 0), A, 0) with Z the
// PARAM za (the ReLU backward rule, tensor/gradient_ruleset.go:153-161); pb/zb likewise for B. A
// prologue is applied in one elementwise pass into the template's workspace before the MFMA kernel.
// wa / wb (dtype f32 only): operand A / B is stored f16 and widened to f32 by that pass (alone, or with
// its prologue); wza / wzb: the mask prologue's Z is stored f16. These are the reference's mixed
// contractions, an f32 adjoint times an f16 weight or activation (tensor/ops.go:74-79).
// variant picks an f16 kernel variant, tile (64/128/256) and kg (k-groups) the f32 tiled kernel's shape.
// M, N and K may be symbolic. PARAMs by epilogue:
//   store      C, A, B                     C = scale*acc
//   bias       C, A, B, bias               C = acc + bias[n]
//   bias_relu  C, A, B, bias               C = relu(acc + bias[n]) (ReLU outputs tagged, see ah_common.h)
//   mask       C, A, B, h                  C = scale*acc where h (a tagged ReLU output) is live, else 0
//   mse (f16)  C, A, B, bias, t; side data5 = per-wave loss partials [ceil(M/32)*ceil(N/32)] f32:
//              P = f16(f16(acc)+bias), C = f16(P - t), partial += (P - t)^2; see mse_loss
//   sgd (f32 master) W', A, B, W       W' = W - lr*(scale*acc)
//   grad       G (f32), A, B               G = scale*acc in f32 whatever the operand dtype (a weight
//              gradient of f16 operands, which the reference computes in f32: tensor/ops.go:74-79)
int template_gemm(const Params &P, TemplateKernel *t) {
    GemmDesc base;
    memset(&base, 0, sizeof base);
    const std::string dt = P.str("dtype", "f32");
    if (dt != "f32" && dt != "f16") return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: dtype %s", dt.c_str());
    base.dtype = dt == "f16" ? GEMM_F16 : GEMM_F32;
    static const std::map<std::string, int> epis = {{"store", EPI_STORE}, {"bias", EPI_BIAS}, {"bias_relu", EPI_BIAS_RELU},
                                                    {"mask", EPI_MASK}, {"mse", EPI_MSE}, {"sgd", EPI_SGD},
                                                    {"grad", kEpiGrad}};
    const std::string epi = P.str("epi", "store");
    auto ei = epis.find(epi);
    if (ei == epis.end()) return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: epilogue %s", epi.c_str());
    const bool grad = ei->second == kEpiGrad;
    base.epi = grad ? EPI_SGD : ei->second;
    if (base.epi == EPI_MSE && base.dtype != GEMM_F16) return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: mse is an f16 epilogue");
    base.ta = (int)P.integer("ta", 0);
    base.tb = (int)P.integer("tb", 0);
    if ((base.ta != 0 && base.ta != 1) || (base.tb != 0 && base.tb != 1)) return set_error(AH_ERR_INVALID, "tmpl gemm: ta/tb are 0 or 1");
    Dim M, N, K;
    GET("M", M, true);
    GET("N", N, true);
    GET("K", K, true);
    base.scale = P.real("scale", 1.0f);
    base.lr = P.real("lr", 0.0f);
    base.variant = (int)P.integer("variant", 0);
    if (base.variant < 0 || base.variant > kGemm16Variants) return set_error(AH_ERR_INVALID, "tmpl gemm: variant %d", base.variant);
    base.tile = (int)P.integer("tile", 0);
    base.kgroups = (int)P.integer("kg", 0);
    if (base.tile != 0 && base.tile != 64 && base.tile != 128 && base.tile != 256)
        return set_error(AH_ERR_INVALID, "tmpl gemm: tile %d", base.tile);
    if (base.kgroups != 0 && !(base.tile != 0 && gemm32_kgroups_ok(base.tile, base.kgroups)))
        return set_error(AH_ERR_INVALID, "tmpl gemm: kg=%d needs a tile that admits it", base.kgroups);
    base.splits = (int)P.integer("splits", 0);
    if (base.splits < 0 || base.splits > 16) return set_error(AH_ERR_INVALID, "tmpl gemm: splits=%d (0..16)", base.splits);
    // dma=i: f32 configuration i of the direct-to-LDS kernel (gemm32d.hip) in place of tile / kg (splits
    // still split K across workgroups)
    const int dma = (int)P.integer("dma", -1);
    if (dma >= 0) {
        if (dma >= kGemm32dConfigs || base.tile || base.kgroups)
            return set_error(AH_ERR_INVALID, "tmpl gemm: dma=%d (0..%d, without tile or kg)", dma, kGemm32dConfigs - 1);
        base.tile = kGemm32dBase + dma;
    }
    const bool swap_ab = P.integer("swap_ab", 0) != 0;
    // PARAM of each role: A, B, bias (or the first epilogue input), and the prologues' mask sources
    const int pA = (int)P.integer("in_a", swap_ab ? 2 : 1), pB = (int)P.integer("in_b", swap_ab ? 1 : 2);
    const int pBias = (int)P.integer("in_bias", 3);
    static const std::map<std::string, int> pros = {{"", 0}, {"relu", 1}, {"mask", 2}};
    auto pa_it = pros.find(P.str("pa", "")), pb_it = pros.find(P.str("pb", ""));
    if (pa_it == pros.end() || pb_it == pros.end()) return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: prologue must be relu or mask");
    int proA = pa_it->second, proB = pb_it->second;
    const int pZa = proA == 2 ? (int)P.integer("za", -1) : -1, pZb = proB == 2 ? (int)P.integer("zb", -1) : -1;
    if ((proA == 2 && pZa < 1) || (proB == 2 && pZb < 1)) return set_error(AH_ERR_INVALID, "tmpl gemm: a mask prologue names its Z PARAM (za/zb)");
    // wa / wb: the operand is stored f16 and widened into an f32 contraction (an f32 adjoint times an f16
    // weight or activation, tensor/ops.go:74-79); wza / wzb: the mask source is stored f16
    const bool wa = P.integer("wa", 0) != 0, wb = P.integer("wb", 0) != 0;
    const bool wza = P.integer("wza", 0) != 0, wzb = P.integer("wzb", 0) != 0;
    if ((wa || wb || wza || wzb) && base.dtype != GEMM_F32) return set_error(AH_ERR_INVALID, "tmpl gemm: wa/wb/wza/wzb widen into an f32 contraction");
    if ((wza && proA != 2) || (wzb && proB != 2)) return set_error(AH_ERR_INVALID, "tmpl gemm: wza/wzb need a mask prologue");
    if (wa && proA == 0) proA = 3;   // widening alone
    if (wb && proB == 0) proB = 3;
    const bool mixed = wa || wb || wza || wzb;
    if ((proA || proB) && (base.epi == EPI_MSE || base.epi == EPI_MASK || base.epi == EPI_SGD))
        return set_error(AH_ERR_UNSUPPORTED, "tmpl gemm: prologues with the store/bias/bias_relu/grad epilogues");
    if (pA < 1 || pB < 1 || pA == pB) return set_error(AH_ERR_INVALID, "tmpl gemm: in_a/in_b must name two input PARAMs");
    int nbuf = (base.epi == EPI_STORE || grad) ? 3 : base.epi == EPI_MSE ? 6 : 4;
    for (int q : {pA + 1, pB + 1, pZa + 1, pZb + 1}) nbuf = std::max(nbuf, q);
    if (base.epi == EPI_BIAS || base.epi == EPI_BIAS_RELU) nbuf = std::max(nbuf, pBias + 1);
    if (base.epi == EPI_MSE) t->side = {{5, true}};
    const int es = base.dtype == GEMM_F16 ? 2 : 4;
    // workspace: the prologue outputs, A' then B' at a 256-byte boundary
    auto ws_layout = [M, N, K, proA, proB, es](int64_t sv, int64_t *offB) -> int64_t {
        const int64_t a = proA ? M.with(sv) * K.with(sv) * es : 0, b = proB ? N.with(sv) * K.with(sv) * es : 0;
        *offB = (a + 255) / 256 * 256;
        return *offB + b;
    };
    if (proA || proB)
        t->workspace = [ws_layout](int64_t sv) -> int64_t { int64_t ob; return ws_layout(sv, &ob); };
    t->bytes = [base, M, N, K, grad, pA, pB, pBias, pZa, pZb, nbuf, es, wa, wb, wza, wzb](int64_t sv) -> std::vector<int64_t> {
        const int64_t m = M.with(sv), n = N.with(sv), k = K.with(sv);
        std::vector<int64_t> b(nbuf, 0);
        b[0] = m * n * ((base.epi == EPI_SGD || grad) ? 4 : es);
        b[pA] = m * k * (wa ? 2 : es);
        b[pB] = n * k * (wb ? 2 : es);
        if (pZa > 0) b[pZa] = m * k * (wza ? 2 : es);
        if (pZb > 0) b[pZb] = n * k * (wzb ? 2 : es);
        switch (base.epi) {
        case EPI_BIAS: case EPI_BIAS_RELU: b[pBias] = n * es; break;
        case EPI_MASK: b[3] = m * n * es; break;
        case EPI_MSE: b[3] = n * es; b[4] = m * n * es; b[5] = (m + 31) / 32 * ((n + 31) / 32) * 4; break;
        case EPI_SGD: if (!grad) b[3] = m * n * 4; break;
        default: break;
        }
        return b;
    };
    const std::string key = t->key;
    t->run = [base, M, N, K, nbuf, grad, key, pA, pB, pBias, proA, proB, pZa, pZb, ws_layout, mixed, wa, wb, wza, wzb](
                 ah_device *d, TemplateKernel *self, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, nbuf)) return rc;
        GemmDesc g = base;
        AT(M, m);
        AT(N, n);
        AT(K, k);
        g.M = (int)m; g.N = (int)n; g.K = (int)k;
        g.A = ptrs[pA];
        g.B = ptrs[pB];
        g.lda = g.ta ? g.M : g.K;
        g.ldb = g.tb ? g.N : g.K;
        g.ldc = g.N;
        g.C = ptrs[0];
        if (proA || proB) {   // prologues into the workspace, then the contraction reads them there
            const int64_t sv = (M.sym || N.sym || K.sym) && ns > 0 ? sc[0] : 0;
            int64_t offB = 0;
            const int64_t bytes = ws_layout(sv, &offB);
            if (int rc = ensure_ws(self, bytes)) return rc;
            const bool f16 = base.dtype == GEMM_F16;
            if (proA) {
                void *dst = self->ws;
                if (mixed) AH_HIP(operand_prologue_f32(ptrs[pA], wa, proA == 2 ? ptrs[pZa] : nullptr, wza, proA, m * k, (float *)dst, d->stream));
                else AH_HIP(operand_prologue(ptrs[pA], proA == 2 ? ptrs[pZa] : nullptr, f16, m * k, dst, d->stream));
                g.A = dst;
            }
            if (proB) {
                void *dst = (char *)self->ws + offB;
                if (mixed) AH_HIP(operand_prologue_f32(ptrs[pB], wb, proB == 2 ? ptrs[pZb] : nullptr, wzb, proB, n * k, (float *)dst, d->stream));
                else AH_HIP(operand_prologue(ptrs[pB], proB == 2 ? ptrs[pZb] : nullptr, f16, n * k, dst, d->stream));
                g.B = dst;
            }
        }
        switch (g.epi) {
        case EPI_BIAS: case EPI_BIAS_RELU: g.bias = ptrs[pBias]; break;
        case EPI_MASK: g.aux = ptrs[3]; g.ldaux = g.N; break;
        case EPI_MSE:
            g.bias = ptrs[3]; g.aux = ptrs[4]; g.ldaux = g.N; g.lossacc = (float *)ptrs[5];
            g.loss_ld = (g.N + 31) / 32;   // deterministic per-wave partials
            break;
        case EPI_SGD: {
            if (grad) {
                // the SGD epilogue on a zeroed f32 array with lr = -1 stores 0 + scale*acc exactly
                AH_HIP(zero_fill(ptrs[0], (long)g.M * g.N * 4, d->stream));
                g.W32 = (float *)ptrs[0];
                g.C = nullptr;
                g.lr = -1.0f;
                break;
            }
            // W' starts as a copy of W and is updated in place by the epilogue
            const size_t bytes = (size_t)g.M * g.N * 4;
            if (ptrs[0] != ptrs[3] && bytes) AH_HIP(hipMemcpyAsync(ptrs[0], ptrs[3], bytes, hipMemcpyDeviceToDevice, d->stream));
            g.W32 = (float *)ptrs[0];
            g.C = nullptr;
            break;
        }
        default: break;
        }
        if (g.M == 0 || g.N == 0) return AH_OK;
        AH_HIP(gemm_dispatch(d, g));
        return AH_OK;
    };
    return AH_OK;
}

// ── reduce ───────────────────────────────────────────────────────────────────────────────────────
// "tmpl:reduce;op=sum|max|sumsq;axis=0|1;M=..;N=..[;scale=s][;dtype=f16][;pa=mask;za=z[;in_a=i][;wza=1]]"
// PARAMs: out (f32), A [M,N]. pa=mask (column sums only): each element enters as Where(Z == max(Z, 0), A, 0)
// with Z [M,N] the PARAM za, stored f16 with wza=1 (the bias gradient of a ReLU layer,
// gradient_ruleset.go:153-161); in_a names A's PARAM (default 1).
int template_reduce(const Params &P, TemplateKernel *t) {
    static const std::map<std::string, int> ops = {{"sum", RED_SUM}, {"max", RED_MAX}, {"sumsq", RED_SUMSQ}};
    auto oi = ops.find(P.str("op", "sum"));
    if (oi == ops.end()) return set_error(AH_ERR_UNSUPPORTED, "tmpl reduce: op %s", P.str("op", "").c_str());
    const int op = oi->second;
    const long axis = P.integer("axis", 1);
    if (axis != 0 && axis != 1) return set_error(AH_ERR_INVALID, "tmpl reduce: axis is 0 or 1");
    Dim M, N;
    GET("M", M, true);
    GET("N", N, true);
    const float scale = P.real("scale", 1.0f);
    const std::string dt = P.str("dtype", "f32");
    if (dt != "f32" && dt != "f16") return set_error(AH_ERR_UNSUPPORTED, "tmpl reduce: dtype %s", dt.c_str());
    const bool f16 = dt == "f16";
    const std::string pa = P.str("pa", "");
    const bool mask = pa == "mask";
    if (!pa.empty() && !mask) return set_error(AH_ERR_UNSUPPORTED, "tmpl reduce: prologue %s", pa.c_str());
    if (mask && (axis != 0 || op != RED_SUM)) return set_error(AH_ERR_UNSUPPORTED, "tmpl reduce: the mask prologue is for column sums");
    const int pA = mask ? (int)P.integer("in_a", 1) : 1, pZ = mask ? (int)P.integer("za", -1) : -1;
    if (mask && (pA < 1 || pA > 2 || pZ < 1 || pZ > 2 || pA == pZ))
        return set_error(AH_ERR_INVALID, "tmpl reduce: in_a and za name PARAMs 1 and 2");
    const bool wz = P.integer("wza", 0) != 0;
    if (wz && !mask) return set_error(AH_ERR_INVALID, "tmpl reduce: wza needs the mask prologue");
    const int nbuf = mask ? 3 : 2;
    const std::string key = t->key;
    t->bytes = [axis, M, N, f16, mask, pA, pZ, wz, nbuf](int64_t sv) -> std::vector<int64_t> {
        const int64_t m = M.with(sv), n = N.with(sv);
        std::vector<int64_t> b(nbuf);
        b[0] = (axis == 0 ? n : m) * 4;
        b[pA] = m * n * (f16 ? 2 : 4);
        if (mask) b[pZ] = m * n * (wz ? 2 : 4);
        return b;
    };
    t->workspace = [axis, M, N](int64_t symv) -> int64_t {
        if (axis != 0) return 0;
        const long m = M.sym ? symv : M.v, n = N.sym ? symv : N.v;
        return m > 0 && n > 0 ? reduce_cols_workspace((int)m, (int)n) * 4 : 0;
    };
    t->run = [op, axis, M, N, scale, f16, key, mask, pA, pZ, wz, nbuf](ah_device *d, TemplateKernel *self, void *const *ptrs,
                                                                      int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, nbuf)) return rc;
        AT(M, m);
        AT(N, n);
        if (axis == 1) {
            AH_HIP(reduce_rows(ptrs[1], f16, (int)m, (int)n, op, scale, (float *)ptrs[0], d->stream));
        } else {
            if (int rc = ensure_ws(self, reduce_cols_workspace((int)m, (int)n) * 4)) return rc;
            AH_HIP(reduce_cols(ptrs[pA], f16, (int)m, (int)n, op, scale, (float *)self->ws, (float *)ptrs[0], d->stream,
                               mask ? ptrs[pZ] : nullptr, wz));
        }
        return AH_OK;
    };
    return AH_OK;
}

// ── softmax cross-entropy ───────────────────────────────────────────────────────────────────────
int template_softmax_ce(const Params &P, TemplateKernel *t) {
    Dim B, C;
    GET("B", B, true);
    GET("C", C, false);
    t->side = {{3, false}};
    t->bytes = [B, C](int64_t sv) -> std::vector<int64_t> {
        const int64_t b = B.with(sv);
        return {b * C.v * 4, b * C.v * 4, b * 4, b * 4};
    };
    const std::string key = t->key;
    t->run = [B, C, key](ah_device *d, TemplateKernel *, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, 4)) return rc;
        AT(B, b);
        const float a = b > 0 ? (float)(-1.0 / (double)b) : 0.0f;
        AH_HIP(softmax_ce((const float *)ptrs[1], (const int32_t *)ptrs[2], (int)b, (int)C.v, a, (float *)ptrs[0],
                          (float *)ptrs[3], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

// ── pooling ─────────────────────────────────────────────────────────────────────────────────────
int template_maxpool(const Params &P, TemplateKernel *t, bool bwd) {
    Dim N, C, H, W, kh, kw, sh, sw;
    GET("N", N, true);
    GET("C", C, false);
    GET("H", H, false);
    GET("W", W, false);
    GET("kh", kh, false);
    GET("kw", kw, false);
    GET("sh", sh, false);
    GET("sw", sw, false);
    if (kh.v < 1 || kw.v < 1 || sh.v < 1 || sw.v < 1 || kh.v > H.v || kw.v > W.v)
        return set_error(AH_ERR_INVALID, "tmpl %s: window %ldx%ld stride %ldx%ld on %ldx%ld", P.name.c_str(), kh.v, kw.v,
                         sh.v, sw.v, H.v, W.v);
    t->bytes = [=](int64_t sv) -> std::vector<int64_t> {
        const int64_t nc = N.with(sv) * C.v, in = nc * H.v * W.v * 4;
        const int64_t out = nc * ((H.v - kh.v) / sh.v + 1) * ((W.v - kw.v) / sw.v + 1) * 4;
        return bwd ? std::vector<int64_t>{in, in, out} : std::vector<int64_t>{out, in};
    };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, bwd ? 3 : 2)) return rc;
        AT(N, n);
        const long nc = n * C.v;
        if (bwd)
            AH_HIP(maxpool_bwd((const float *)ptrs[1], (const float *)ptrs[2], nc, (int)H.v, (int)W.v, (int)kh.v, (int)kw.v,
                               (int)sh.v, (int)sw.v, (float *)ptrs[0], d->stream));
        else
            AH_HIP(maxpool_fwd((const float *)ptrs[1], nc, (int)H.v, (int)W.v, (int)kh.v, (int)kw.v, (int)sh.v, (int)sw.v,
                               (float *)ptrs[0], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

int template_pool_relu_bwd(const Params &P, TemplateKernel *t) {
    Dim N, C, H;
    GET("N", N, true);
    GET("C", C, false);
    GET("H", H, false);
    if (H.v % 2) return set_error(AH_ERR_INVALID, "tmpl pool_relu_bwd: H must be even");
    t->bytes = [=](int64_t sv) -> std::vector<int64_t> {
        const int64_t full = N.with(sv) * C.v * H.v * H.v * 4, half = full / 4;
        return {full, half, full, half};
    };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, 4)) return rc;
        AT(N, n);
        AH_HIP(pool_relu_bwd((const float *)ptrs[1], (const float *)ptrs[2], (const float *)ptrs[3], (int)(n * C.v), (int)H.v,
                             (float *)ptrs[0], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

// ── convolution (3x3, padding 1, stride 1) ──────────────────────────────────────────────────────
enum ConvKind { CONV_FWD, CONV_FWD_POOL, CONV_BWD_X, CONV_BWD_W, CONV_BWD_B };

int template_conv(const Params &P, TemplateKernel *t, ConvKind kind) {
    Dim N, Ci, Co, H;
    GET("N", N, true);
    GET("Co", Co, false);
    GET("H", H, false);
    if (kind != CONV_BWD_B) GET("Ci", Ci, false);
    if (kind == CONV_FWD_POOL && H.v % 2) return set_error(AH_ERR_INVALID, "tmpl conv2d_relu_pool: H must be even");
    const int relu = (int)P.integer("relu", 0);
    if (kind == CONV_FWD_POOL) t->side = {{4, false}};
    t->bytes = [=](int64_t sv) -> std::vector<int64_t> {
        const int64_t n = N.with(sv), hh = H.v * H.v, xi = n * Ci.v * hh * 4, yo = n * Co.v * hh * 4;
        const int64_t w = Co.v * Ci.v * 9 * 4, b = Co.v * 4;
        switch (kind) {
        case CONV_FWD: return {yo, xi, w, b};
        case CONV_FWD_POOL: return {yo / 4, xi, w, b, yo};
        case CONV_BWD_X: return {xi, yo, w};
        case CONV_BWD_W: return {w, xi, yo};
        default: return {b, yo};
        }
    };
    if (kind == CONV_BWD_W)
        t->workspace = [N, Ci, Co, H](int64_t symv) -> int64_t {
            const long n = N.sym ? symv : N.v;
            return n > 0 ? (int64_t)conv_bwd_w_splits((int)n, (int)Ci.v, (int)H.v, (int)Co.v) * Co.v * Ci.v * 10 * 4 : 0;
        };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *self, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        static const int want[] = {4, 5, 3, 3, 2};
        if (int rc = need(key.c_str(), n_ptrs, want[kind])) return rc;
        AT(N, n);
        const float *in1 = (const float *)ptrs[1], *in2 = n_ptrs > 2 ? (const float *)ptrs[2] : nullptr;
        switch (kind) {
        case CONV_FWD:
            AH_HIP(conv3x3_fwd(in1, (int)n, (int)Ci.v, (int)H.v, in2, (const float *)ptrs[3], (int)Co.v, relu, (float *)ptrs[0], d->stream));
            break;
        case CONV_FWD_POOL:
            AH_HIP(conv_fwd_relu_pool(in1, (int)n, (int)Ci.v, (int)H.v, in2, (const float *)ptrs[3], (int)Co.v,
                                      (float *)ptrs[4], (float *)ptrs[0], d->stream));
            break;
        case CONV_BWD_X:
            AH_HIP(conv_bwd_x(in1, in2, (int)n, (int)Ci.v, (int)H.v, (int)Co.v, (float *)ptrs[0], d->stream));
            break;
        case CONV_BWD_W: {
            const int64_t bytes = (int64_t)conv_bwd_w_splits((int)n, (int)Ci.v, (int)H.v, (int)Co.v) * Co.v * Ci.v * 10 * 4;
            if (int rc = ensure_ws(self, bytes)) return rc;
            AH_HIP(conv_bwd_w_partial(in1, in2, (int)n, (int)Ci.v, (int)H.v, (int)Co.v, (float *)self->ws, d->stream));
            AH_HIP(conv_bwd_w_finalize((const float *)self->ws, (int)n, (int)Ci.v, (int)H.v, (int)Co.v, nullptr, nullptr, 0.0f,
                                       (float *)ptrs[0], nullptr, d->stream));
            break;
        }
        case CONV_BWD_B:
            AH_HIP(conv_bias_grad(in1, (int)n, (int)Co.v, (int)(H.v * H.v), (float *)ptrs[0], d->stream));
            break;
        }
        return AH_OK;
    };
    return AH_OK;
}

// ── elementwise SGD, MSE loss, config-5 chain ───────────────────────────────────────────────────
int template_sgd(const Params &P, TemplateKernel *t) {
    Dim n;
    GET("n", n, true);
    const float lr = P.real("lr", 0.0f), scale = P.real("scale", 1.0f);
    t->bytes = [n](int64_t sv) -> std::vector<int64_t> { const int64_t b = n.with(sv) * 4; return {b, b, b}; };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, 3)) return rc;
        AT(n, len);
        AH_HIP(sgd_out((const float *)ptrs[1], (const float *)ptrs[2], len, lr, scale, (float *)ptrs[0], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

int template_mse_loss(const Params &P, TemplateKernel *t) {
    Dim parts;
    GET("parts", parts, true);
    const float scale = P.real("scale", 1.0f);
    t->bytes = [parts](int64_t sv) -> std::vector<int64_t> { return {4, parts.with(sv) * 4}; };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *, void *const *ptrs, int32_t n_ptrs, const int32_t *sc, int32_t ns) -> int {
        if (int rc = need(key.c_str(), n_ptrs, 2)) return rc;
        AT(parts, np);
        AH_HIP(mse_loss((const float *)ptrs[1], np, scale, (float *)ptrs[0], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

int template_chain(const Params &P, TemplateKernel *t) {
    Dim R, Cc;
    GET("R", R, false);
    GET("Cc", Cc, false);
    if (R.v <= 0 || Cc.v <= 0 || Cc.v % 4) return set_error(AH_ERR_INVALID, "tmpl chain: Cc must be a positive multiple of 4");
    t->side = {{3, false}, {4, false}};
    t->bytes = [R, Cc](int64_t) -> std::vector<int64_t> {
        const int64_t x = R.v * Cc.v * 4;
        return {x, x, Cc.v * 4, Cc.v * 4, 4};
    };
    t->workspace = [R, Cc](int64_t) -> int64_t { return chain_workspace_floats((int)R.v, (int)Cc.v) * 4; };
    const std::string key = t->key;
    t->run = [=](ah_device *d, TemplateKernel *self, void *const *ptrs, int32_t n_ptrs, const int32_t *, int32_t) -> int {
        if (int rc = need(key.c_str(), n_ptrs, 5)) return rc;
        if (int rc = ensure_ws(self, chain_workspace_floats((int)R.v, (int)Cc.v) * 4)) return rc;
        AH_HIP(chain_step((const float *)ptrs[1], (const float *)ptrs[2], (int)R.v, (int)Cc.v, (float *)self->ws,
                          (float *)ptrs[0], (float *)ptrs[3], (float *)ptrs[4], d->stream));
        return AH_OK;
    };
    return AH_OK;
}

}  // namespace

TemplateKernel::~TemplateKernel() {
    if (ws) (void)hipFree(ws);
}

int template_prepare(TemplateKernel *t, int64_t symval) {
    if (!t->workspace) return AH_OK;
    return ensure_ws(t, t->workspace(symval));
}

int template_create(const std::string &source, TemplateKernel **out) {
    Params P;
    P.kv = template_key_params(source, &P.name);
    auto *t = new TemplateKernel();
    t->key = source;
    t->name = P.name;
    int rc;
    if (P.name == "gemm") rc = template_gemm(P, t);
    else if (P.name == "reduce") rc = template_reduce(P, t);
    else if (P.name == "softmax_ce") rc = template_softmax_ce(P, t);
    else if (P.name == "maxpool2d") rc = template_maxpool(P, t, false);
    else if (P.name == "maxpool2d_bwd") rc = template_maxpool(P, t, true);
    else if (P.name == "pool_relu_bwd") rc = template_pool_relu_bwd(P, t);
    else if (P.name == "conv2d") rc = template_conv(P, t, CONV_FWD);
    else if (P.name == "conv2d_relu_pool") rc = template_conv(P, t, CONV_FWD_POOL);
    else if (P.name == "conv2d_bwd_x") rc = template_conv(P, t, CONV_BWD_X);
    else if (P.name == "conv2d_bwd_w") rc = template_conv(P, t, CONV_BWD_W);
    else if (P.name == "conv2d_bwd_b") rc = template_conv(P, t, CONV_BWD_B);
    else if (P.name == "sgd") rc = template_sgd(P, t);
    else if (P.name == "mse_loss") rc = template_mse_loss(P, t);
    else if (P.name == "chain") rc = template_chain(P, t);
    else rc = set_error(AH_ERR_UNSUPPORTED, "unknown template '%s'", P.name.c_str());
    if (rc != AH_OK) {
        delete t;
        return rc;
    }
    *out = t;
    return AH_OK;
}

}  // namespace ah
