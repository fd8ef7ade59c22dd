// wgsl_match.cpp — selects a hand-written contraction template for a WGSL kernel the reference's
// codegen rendered as a plain REDUCE(ADD, MUL(load, load)) (codegen/lower.go:98-550 rendered by
// codegen/wgsl.go:36-238): the role the north star gives a rewrite/ pattern in front of the renderer,
// taken at the boundary where the backend receives the kernel (a cached ExecItem carries only its WGSL,
// schedule/cache.go:69-100).
//
// The kernel must have exactly this shape (any order of the two loads and of the product's factors):
//   let rA: i32 = i32(<expr of flat_gid_x>);  if (rA >= M) { return; }    (the output axes, GIDVar)
//   var accI: f32 = 0.0;
//   for (var rK: i32 = 0; rK < K; rK++) {
//     let tX: f32 = dataP[<index>];  let tY: f32 = dataQ[<index>];
//     accI = accI + (tX * tY);
//   }
//   data0[<index>] = accI;
// with three f32 bindings and no symbolic parameters, or with a fourth, data3, holding a bias b[n] that
// is added to accI before the store (let tB: f32 = data3[<index>]; then (accI + tB) or (tB + accI),
// as a let or in the store): the Linear forward epilogue, "tmpl:gemm;epi=bias", the same f32 add. The index expressions are not parsed for
// structure: they are evaluated (the scheduler's unsimplified chains of / and % included, as integer
// arithmetic) at every point of each axis and at sampled points of the whole index space, and must be
// affine there with zero offset. The coefficients then give the contraction: C [M,N] row-major, A read
// K-contiguous ([M,K]) or MN-contiguous ([K,M]), B likewise, which is "tmpl:gemm" (templates.cpp) with
// ta/tb and, when the first-bound input is B, swap_ab=1. Anything else (and any axis of more than 2^16
// points) is left to the WGSL renderer.
#include <ctype.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

namespace ah {
namespace {

std::string trim(const std::string &s) {
    size_t a = s.find_first_not_of(" \t\r"), b = s.find_last_not_of(" \t\r");
    return a == std::string::npos ? std::string() : s.substr(a, b - a + 1);
}

// Integer expression over the WGSL index subset: literals (optional u/i suffix), rN / flat_gid_x names,
// + - * / % (truncating, as WGSL i32/u32 on the non-negative values here), parentheses, i32(...) and
// u32(...) casts (identity). Returns false on anything else or on division by zero.
struct Expr {
    const char *p;
    const std::map<std::string, int64_t> &vars;
    bool ok = true;
    Expr(const char *s, const std::map<std::string, int64_t> &v) : p(s), vars(v) {}
    void ws() { while (*p == ' ') p++; }
    int64_t primary() {
        ws();
        if (*p == '(') {
            p++;
            int64_t v = sum();
            ws();
            if (*p != ')') { ok = false; return 0; }
            p++;
            return v;
        }
        if (isdigit((unsigned char)*p)) {
            int64_t v = 0;
            while (isdigit((unsigned char)*p)) v = v * 10 + (*p++ - '0');
            if (*p == 'u' || *p == 'i') p++;
            return v;
        }
        if (isalpha((unsigned char)*p) || *p == '_') {
            std::string name;
            while (isalnum((unsigned char)*p) || *p == '_') name += *p++;
            ws();
            if ((name == "i32" || name == "u32") && *p == '(') return primary();
            auto it = vars.find(name);
            if (it == vars.end()) { ok = false; return 0; }
            return it->second;
        }
        ok = false;
        return 0;
    }
    int64_t product() {
        int64_t v = primary();
        for (;;) {
            ws();
            char c = *p;
            if (c != '*' && c != '/' && c != '%') return v;
            p++;
            int64_t r = primary();
            if (c == '*') v *= r;
            else if (r == 0) { ok = false; return 0; }
            else v = c == '/' ? v / r : v % r;
        }
    }
    int64_t sum() {
        int64_t v = product();
        for (;;) {
            ws();
            char c = *p;
            if (c != '+' && c != '-') return v;
            p++;
            int64_t r = product();
            v = c == '+' ? v + r : v - r;
        }
    }
};

bool eval(const std::string &e, const std::map<std::string, int64_t> &vars, int64_t *out) {
    Expr x(e.c_str(), vars);
    int64_t v = x.sum();
    x.ws();
    if (!x.ok || *x.p) return false;
    *out = v;
    return true;
}

bool starts(const std::string &s, const char *pre) { return s.compare(0, strlen(pre), pre) == 0; }

// "let NAME: TYPE = EXPR;" -> name, type, expr
bool parse_let(const std::string &s, std::string *name, std::string *type, std::string *expr) {
    if (!starts(s, "let ") || s.back() != ';') return false;
    size_t c = s.find(':'), e = s.find('=');
    if (c == std::string::npos || e == std::string::npos || e < c) return false;
    *name = trim(s.substr(4, c - 4));
    *type = trim(s.substr(c + 1, e - c - 1));
    *expr = trim(s.substr(e + 1, s.size() - e - 2));
    return true;
}

// "dataP[IDX]" -> P, IDX
bool parse_load(const std::string &e, int *buf, std::string *idx) {
    if (!starts(e, "data") || e.back() != ']') return false;
    size_t b = e.find('[');
    if (b == std::string::npos) return false;
    const std::string num = e.substr(4, b - 4);
    if (num.empty() || num.find_first_not_of("0123456789") != std::string::npos) return false;
    *buf = atoi(num.c_str());
    *idx = e.substr(b + 1, e.size() - b - 2);
    return true;
}

struct Axis {
    std::string name, expr;   // rN and its GIDVar expression of flat_gid_x
    int64_t range = 1;
};

// Affine coefficients of idx over (m, n, k) with zero offset, checked on every point of each axis and
// on sampled points of the whole space. vars holds the axis values used for the evaluation.
bool affine(const std::string &idx, const std::string vn[3], const int64_t range[3], int64_t coef[3]) {
    std::map<std::string, int64_t> v;
    for (int a = 0; a < 3; a++) v[vn[a]] = 0;
    v["flat_gid_x"] = 0;
    auto at = [&](int64_t x0, int64_t x1, int64_t x2, int64_t *o) {
        v[vn[0]] = x0; v[vn[1]] = x1; v[vn[2]] = x2;
        return eval(idx, v, o);
    };
    int64_t base;
    if (!at(0, 0, 0, &base) || base != 0) return false;
    for (int a = 0; a < 3; a++) {
        int64_t x[3] = {0, 0, 0}, o;
        coef[a] = 0;
        if (range[a] > 1) {
            x[a] = 1;
            if (!at(x[0], x[1], x[2], &o)) return false;
            coef[a] = o;
        }
        for (int64_t i = 0; i < range[a]; i++) {   // every point of the axis
            x[a] = i;
            if (!at(x[0], x[1], x[2], &o) || o != coef[a] * i) return false;
        }
    }
    uint64_t h = 0x9e3779b97f4a7c15ull;
    for (int s = 0; s < 4096; s++) {                // sampled points of the whole space
        int64_t x[3], o;
        for (int a = 0; a < 3; a++) {
            h ^= h >> 12; h ^= h << 25; h ^= h >> 27;
            x[a] = (int64_t)((h * 2685821657736338717ull) >> 33) % range[a];
        }
        if (s < 8)                                  // and the corners
            for (int a = 0; a < 3; a++) x[a] = (s >> a) & 1 ? range[a] - 1 : 0;
        if (!at(x[0], x[1], x[2], &o) || o != coef[0] * x[0] + coef[1] * x[1] + coef[2] * x[2]) return false;
    }
    return true;
}

}  // namespace

bool wgsl_match_contraction(const std::string &src, std::string *key) {
    std::vector<std::string> L;
    {
        size_t a = 0;
        while (a <= src.size()) {
            size_t b = src.find('\n', a);
            if (b == std::string::npos) b = src.size();
            std::string t = trim(src.substr(a, b - a));
            if (!t.empty()) L.push_back(t);
            a = b + 1;
        }
    }
    // bindings: data0..2, all f32, nothing else bound
    int nb = 0;
    size_t i = 0;
    for (; i < L.size() && !starts(L[i], "@compute"); i++) {
        if (starts(L[i], "enable ")) continue;
        if (!starts(L[i], "@group(0) @binding(")) return false;   // a params block: symbolic, not matched
        char want[96];
        snprintf(want, sizeof want, "var<storage, %s> data%d: array<f32>;", nb == 0 ? "read_write" : "read", nb);
        if (L[i].find(want) == std::string::npos) return false;
        nb++;
    }
    if ((nb != 3 && nb != 4) || i == L.size()) return false;
    // the fixed preamble ends with "let gid_x = ..."
    for (; i < L.size() && !starts(L[i], "let gid_x ="); i++)
        if (L[i].find("var<workgroup>") != std::string::npos) return false;
    if (i == L.size()) return false;
    i++;
    // output axes
    std::vector<Axis> axes;
    std::string name, type, expr;
    while (i < L.size() && starts(L[i], "let r") && parse_let(L[i], &name, &type, &expr) && type == "i32") {
        Axis ax{name, expr, 1};
        i++;
        char guard[64];
        snprintf(guard, sizeof guard, "if (%s >= ", name.c_str());
        if (i < L.size() && starts(L[i], guard)) {
            const std::string rest = L[i].substr(strlen(guard));
            const size_t close = rest.find(')');
            if (close == std::string::npos || trim(rest.substr(close)) != ") { return; }") return false;
            ax.range = atoll(rest.substr(0, close).c_str());
            if (ax.range < 1) return false;
            i++;
        }
        axes.push_back(ax);
    }
    // accumulator, loop, two loads, the multiply-add, loop end, [bias], store, function end
    if (i + 8 > L.size()) return false;
    std::string acc;
    {
        const std::string &s = L[i++];
        const size_t colon = s.find(':');
        if (!starts(s, "var acc") || colon == std::string::npos || s.substr(colon) != ": f32 = 0.0;") return false;
        acc = trim(s.substr(4, colon - 4));
    }
    std::string kv;
    int64_t K = 0;
    {
        const std::string &s = L[i++];
        char a[32], b[32], c[32];
        long long k = 0;
        if (sscanf(s.c_str(), "for (var %31[^:]: i32 = 0; %31s < %lld; %31[^+]++) {", a, b, &k, c) != 4) return false;
        kv = a;
        if (kv != b || kv != c || k < 1) return false;
        K = k;
    }
    int buf[2];
    std::string tname[2], idx[2];
    for (int j = 0; j < 2; j++) {
        if (!parse_let(L[i++], &tname[j], &type, &expr) || type != "f32" || !parse_load(expr, &buf[j], &idx[j])) return false;
    }
    {
        const std::string a = acc + " = " + acc + " + (" + tname[0] + " * " + tname[1] + ");";
        const std::string b = acc + " = " + acc + " + (" + tname[1] + " * " + tname[0] + ");";
        if (L[i] != a && L[i] != b) return false;
        i++;
    }
    if (L[i++] != "}") return false;
    // optional bias epilogue (Linear forward, acc + b[n], codegen/wgsl.go:270 renders the add as
    // "(a + b)"): a load of data3, then the sum as a let or inline in the store
    std::string bname, bidx, sname;
    while (i + 2 < L.size()) {
        std::string bn, bt, be, bi;
        int bb = -1;
        if (!parse_let(L[i], &bn, &bt, &be) || bt != "f32") return false;
        if (bname.empty() && parse_load(be, &bb, &bi) && bb == 3) {
            bname = bn;
            bidx = bi;
        } else if (!bname.empty() && sname.empty() && (be == "(" + acc + " + " + bname + ")" || be == "(" + bname + " + " + acc + ")")) {
            sname = bn;
        } else {
            return false;
        }
        i++;
    }
    if (L.size() - i != 2) return false;
    std::string cidx;
    {
        const std::string &s = L[i++];
        std::vector<std::string> vals;   // what the store may write
        if (bname.empty()) vals = {acc};
        else if (!sname.empty()) vals = {sname};
        else vals = {"(" + acc + " + " + bname + ")", "(" + bname + " + " + acc + ")"};
        bool ok = false;
        for (const std::string &v : vals) {
            const std::string tail = "] = " + v + ";";
            if (starts(s, "data0[") && s.size() > tail.size() + 6 && s.compare(s.size() - tail.size(), tail.size(), tail) == 0) {
                cidx = s.substr(6, s.size() - 6 - tail.size());
                ok = true;
            }
        }
        if (!ok) return false;
    }
    if (L[i] != "}") return false;
    if (!((buf[0] == 1 && buf[1] == 2) || (buf[0] == 2 && buf[1] == 1))) return false;
    if ((nb == 4) != !bname.empty()) return false;   // data3 is bound exactly when it is the bias
    // two output axes with more than one point (others are size 1 and must not move any index)
    std::vector<const Axis *> live;
    for (const Axis &a : axes)
        if (a.range > 1) live.push_back(&a);
    if (live.size() != 2) return false;
    // axis values are what the loads see; the loads and the store are evaluated over (axis0, axis1, k)
    // with the other axes at 0 (their only value)
    const std::string vn[3] = {live[0]->name, live[1]->name, kv};
    const int64_t range[3] = {live[0]->range, live[1]->range, K};
    // every point of each axis is evaluated below: axes beyond 2^16 points are left to the rendering
    for (int a = 0; a < 3; a++)
        if (range[a] > (1 << 16)) return false;
    for (const Axis &a : axes)
        if (a.name == kv) return false;
    int64_t ca[3], cb[3], cc[3];
    if (!affine(idx[0], vn, range, ca) || !affine(idx[1], vn, range, cb) || !affine(cidx, vn, range, cc)) return false;
    // each output axis must be one of the GIDVar forms codegen/wgsl.go:150-167 emits for a concrete
    // range: i32(flat_gid_x % R) or i32((flat_gid_x / S) % R), with R the axis's guard
    for (const Axis *a : live) {
        long long r = 0, st = 0;
        char tail[8] = {0};
        const bool plain = sscanf(a->expr.c_str(), "i32(flat_gid_x %% %lldu)%7s", &r, tail) == 1;
        const bool strided = !plain && sscanf(a->expr.c_str(), "i32((flat_gid_x / %lldu) %% %lldu)%7s", &st, &r, tail) == 2 && st > 0;
        if ((!plain && !strided) || r != a->range) return false;
    }
    // roles: C = cm*m + n (row-major [M,N]); A depends on m and k, B on n and k
    int im, in;
    if (cc[1] == 1 && cc[0] == range[1] && cc[2] == 0) { im = 0; in = 1; }
    else if (cc[0] == 1 && cc[1] == range[0] && cc[2] == 0) { im = 1; in = 0; }
    else return false;
    const int64_t M = range[im], N = range[in];
    int ia = -1;   // which load is A
    for (int j = 0; j < 2; j++) {
        const int64_t *c = j == 0 ? ca : cb;
        if (c[in] == 0 && (c[im] != 0 || M == 1)) ia = j;
    }
    if (ia < 0) return false;
    const int64_t *A = ia == 0 ? ca : cb, *B = ia == 0 ? cb : ca;
    if (B[im] != 0) return false;
    int ta, tb;
    if (A[2] == 1 && A[im] == K) ta = 0;
    else if (A[im] == 1 && A[2] == M) ta = 1;
    else return false;
    if (B[2] == 1 && B[in] == K) tb = 0;
    else if (B[in] == 1 && B[2] == N) tb = 1;
    else return false;
    if (!bname.empty()) {   // the bias index must be n itself
        int64_t cbias[3];
        if (!affine(bidx, vn, range, cbias) || cbias[in] != 1 || cbias[im] != 0 || cbias[2] != 0) return false;
    }
    const bool swap = buf[ia] == 2;
    char k[160];
    snprintf(k, sizeof k, "tmpl:gemm;dtype=f32;epi=%s;ta=%d;tb=%d;M=%lld;N=%lld;K=%lld%s", bname.empty() ? "store" : "bias",
             ta, tb, (long long)M, (long long)N, (long long)K, swap ? ";swap_ab=1" : "");
    *key = k;
    return true;
}

}  // namespace ah
