// wgsl_match.cpp — selects a hand-written template for a WGSL kernel the reference's codegen rendered
// (codegen/lower.go:98-719 lowered, codegen/wgsl.go:41-386 rendered): the role the north star gives a
// rewrite/ pattern in front of the renderer, taken at the boundary where the backend receives the kernel
// (a cached ExecItem carries only its WGSL, schedule/cache.go:69-100).
//
// The lowering emits one `let tN: T = ...;` per ALU node and per load (emitALU / emitIndex), the output
// axes as GIDVar lets of flat_gid_x/y/z with `if (rN >= R) { return; }` guards (symbolic axes as
// `i32(flat_gid_x / S)` with a params_n bounds check), one accumulator per reduce
// (`var accI: T = identity;` and `accI = accI + e;` or `accI = max(accI, e);` inside one loop per reduce
// range, bounds `i32(params_n.n0)` when symbolic), f16 reduces widened to f32 in the loop and narrowed
// after it as `f16(accI)`, and one store `data0[(u32(r0) * S) + u32(r1)] = v;`. The matcher parses that
// body, substitutes every let into the expression tree it names, and recognises two families:
//
//   contraction  REDUCE(ADD, MUL(opA, opB)) over one loop (f32, f16, or f32 with f16 operands widened in
//                the loop, which the key marks wa / wb / wza / wzb), where an operand is a load, a ReLU prologue
//                max(load, 0.0), or the ReLU-backward mask prologue select(0.0, adj, z == max(z, 0.0))
//                (tensor/gradient_ruleset.go:153-161 with ReLU = Maximum(x, 0), tensor/nn/nn.go:111-114);
//                stored as acc, f16(acc), c*acc, acc + bias[n] (f16: f16(acc) + bias) or
//                max(acc + bias[n], 0.0) (f16: max(f16(acc) + bias, 0.0))  ->  "tmpl:gemm" with ta/tb,
//                prologues pa/pb and PARAM roles;
//   reduction    REDUCE(ADD|MAX, load) over the innermost or the outermost axis of a 2-D buffer (or all
//                of a 1-D one), or REDUCE(ADD) of the ReLU-backward mask prologue down a column (a ReLU
//                layer's bias gradient, the mask source at the same element, f16 sources widened),
//                stored as acc or c*acc into f32  ->  "tmpl:reduce" (pa=mask for the masked form).
//
// Index expressions are not matched as text: they are evaluated as integer arithmetic (the scheduler's
// unsimplified chains of / and % included) at every point of each axis and at sampled points of the
// whole space, and must be affine there with zero offset. A kernel with a symbolic batch is analysed at
// two bindings and selected only when both give the same template (its symbolic ranges become "sym").
// Anything else (and any axis of more than 2^16 points) is left to the WGSL renderer (wgsl.cpp).
#include <ctype.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ah {
namespace {

std::string trim(const std::string &s) {
    size_t a = s.find_first_not_of(" \t\r"), b = s.find_last_not_of(" \t\r");
    return a == std::string::npos ? std::string() : s.substr(a, b - a + 1);
}
bool starts(const std::string &s, const char *pre) { return s.compare(0, strlen(pre), pre) == 0; }

// ── expression trees ────────────────────────────────────────────────────────────────────────────
struct Node;
using P = std::shared_ptr<const Node>;
struct Node {
    enum Kind { NUM, VAR, BIN, CALL, LOAD, NEG } k;
    std::string s;      // VAR name, BIN operator, CALL function (with its <T> for bitcast)
    double num = 0;     // NUM value
    bool isint = false; // NUM written without a decimal point (an index / integer literal)
    int buf = -1;       // LOAD: binding index
    std::vector<P> a;   // operands
};

P mk(Node::Kind k, std::string s = "", std::vector<P> a = {}) {
    auto n = std::make_shared<Node>();
    n->k = k;
    n->s = std::move(s);
    n->a = std::move(a);
    return n;
}

bool same(const P &x, const P &y) {
    if (x->k != y->k || x->s != y->s || x->buf != y->buf || x->a.size() != y->a.size()) return false;
    if (x->k == Node::NUM && x->num != y->num) return false;
    for (size_t i = 0; i < x->a.size(); i++)
        if (!same(x->a[i], y->a[i])) return false;
    return true;
}

// Recursive-descent parser over the rendered expression subset. Names bound by `let` are replaced by
// their (already substituted) trees as they are read.
struct Parser {
    const char *p;
    const std::map<std::string, P> &lets;
    bool ok = true;
    Parser(const char *s, const std::map<std::string, P> &l) : p(s), lets(l) {}
    void ws() { while (*p == ' ') p++; }
    bool eat(const char *t) {
        ws();
        const size_t n = strlen(t);
        if (strncmp(p, t, n) != 0) return false;
        p += n;
        return true;
    }
    P fail() { ok = false; return mk(Node::NUM); }
    P primary() {
        ws();
        if (*p == '(') {
            p++;
            P v = cmp();
            if (!eat(")")) return fail();
            return v;
        }
        if (*p == '-') {
            p++;
            P v = primary();
            if (v->k == Node::NUM) {
                auto n = std::make_shared<Node>(*v);
                n->num = -n->num;
                return n;
            }
            return mk(Node::NEG, "", {v});
        }
        if (isdigit((unsigned char)*p) || (*p == '.' && isdigit((unsigned char)p[1]))) {
            const char *q = p;
            auto n = std::make_shared<Node>();
            n->k = Node::NUM;
            if (p[0] == '0' && (p[1] == 'x' || p[1] == 'X')) {
                n->num = (double)strtoull(p, (char **)&q, 16);
                n->isint = true;
            } else {
                n->num = strtod(p, (char **)&q);
                n->isint = true;
                for (const char *c = p; c < q; c++)
                    if (*c == '.' || *c == 'e' || *c == 'E') n->isint = false;
            }
            p = q;
            if (*p == 'u' || *p == 'i' || *p == 'f' || *p == 'h') p++;
            return n;
        }
        if (isalpha((unsigned char)*p) || *p == '_') {
            std::string name;
            while (isalnum((unsigned char)*p) || *p == '_') name += *p++;
            if (name == "params_n" && *p == '.') {
                p++;
                std::string f;
                while (isalnum((unsigned char)*p)) f += *p++;
                return mk(Node::VAR, "params_n." + f);
            }
            if (name == "bitcast" && *p == '<') {
                const char *e = strchr(p, '>');
                if (!e) return fail();
                name += std::string(p, e + 1);
                p = e + 1;
            }
            ws();
            if (starts(name, "data") && *p == '[') {
                const std::string num = name.substr(4);
                if (num.empty() || num.find_first_not_of("0123456789") != std::string::npos) return fail();
                p++;
                P idx = cmp();
                if (!eat("]")) return fail();
                auto n = mk(Node::LOAD, "", {idx});
                std::const_pointer_cast<Node>(n)->buf = atoi(num.c_str());
                return n;
            }
            if (*p == '(') {
                p++;
                std::vector<P> args;
                ws();
                if (*p != ')')
                    for (;;) {
                        args.push_back(cmp());
                        if (eat(",")) continue;
                        break;
                    }
                if (!eat(")")) return fail();
                return mk(Node::CALL, name, args);
            }
            auto it = lets.find(name);
            if (it != lets.end()) return it->second;
            return mk(Node::VAR, name);
        }
        return fail();
    }
    P product() {
        P v = primary();
        for (;;) {
            ws();
            const char c = *p;
            if ((c != '*' && c != '/' && c != '%') || !ok) return v;
            p++;
            v = mk(Node::BIN, std::string(1, c), {v, primary()});
        }
    }
    P sum() {
        P v = product();
        for (;;) {
            ws();
            const char c = *p;
            if ((c != '+' && c != '-') || !ok) return v;
            p++;
            v = mk(Node::BIN, std::string(1, c), {v, product()});
        }
    }
    P cmp() {
        P v = sum();
        ws();
        static const char *ops[] = {"==", "!=", "<=", ">=", "<", ">"};
        for (const char *o : ops)
            if (strncmp(p, o, strlen(o)) == 0) {
                p += strlen(o);
                return mk(Node::BIN, o, {v, sum()});
            }
        return v;
    }
};

bool parse_expr(const std::string &e, const std::map<std::string, P> &lets, P *out) {
    Parser ps(e.c_str(), lets);
    *out = ps.cmp();
    ps.ws();
    return ps.ok && *ps.p == 0;
}

// Integer value of an index tree (i32/u32 casts are the identity on the non-negative values here).
bool ieval(const P &n, const std::map<std::string, int64_t> &env, int64_t *o) {
    switch (n->k) {
    case Node::NUM:
        if (!n->isint) return false;
        *o = (int64_t)n->num;
        return true;
    case Node::VAR: {
        auto it = env.find(n->s);
        if (it == env.end()) return false;
        *o = it->second;
        return true;
    }
    case Node::NEG: {
        int64_t v;
        if (!ieval(n->a[0], env, &v)) return false;
        *o = -v;
        return true;
    }
    case Node::CALL:
        if ((n->s == "i32" || n->s == "u32") && n->a.size() == 1) return ieval(n->a[0], env, o);
        return false;
    case Node::BIN: {
        int64_t x, y;
        if (!ieval(n->a[0], env, &x) || !ieval(n->a[1], env, &y)) return false;
        const char c = n->s[0];
        if (n->s.size() != 1) return false;
        if (c == '+') *o = x + y;
        else if (c == '-') *o = x - y;
        else if (c == '*') *o = x * y;
        else if (y == 0) return false;
        else if (c == '/') *o = x / y;
        else if (c == '%') *o = x % y;
        else return false;
        return true;
    }
    default: return false;
    }
}

// Affine coefficients of idx over the variables vn (ranges rg) with zero offset, checked on every point of
// each axis and on sampled points of the whole space (the corners first).
bool affine(const P &idx, const std::vector<std::string> &vn, const std::vector<int64_t> &rg, std::vector<int64_t> *coef) {
    const size_t d = vn.size();
    std::map<std::string, int64_t> env;
    for (auto &v : vn) env[v] = 0;
    auto at = [&](const std::vector<int64_t> &x, int64_t *o) {
        for (size_t a = 0; a < d; a++) env[vn[a]] = x[a];
        return ieval(idx, env, o);
    };
    std::vector<int64_t> x(d, 0);
    int64_t o;
    if (!at(x, &o) || o != 0) return false;
    coef->assign(d, 0);
    for (size_t a = 0; a < d; a++) {
        std::vector<int64_t> y(d, 0);
        if (rg[a] > 1) {
            y[a] = 1;
            if (!at(y, &o)) return false;
            (*coef)[a] = o;
        }
        for (int64_t i = 0; i < rg[a]; i++) {
            y[a] = i;
            if (!at(y, &o) || o != (*coef)[a] * i) return false;
        }
    }
    uint64_t h = 0x9e3779b97f4a7c15ull;
    for (int s = 0; s < 4096; s++) {
        for (size_t a = 0; a < d; a++) {
            h ^= h >> 12; h ^= h << 25; h ^= h >> 27;
            x[a] = (int64_t)((h * 2685821657736338717ull) >> 33) % rg[a];
            if (s < (1 << d)) x[a] = (s >> a) & 1 ? rg[a] - 1 : 0;
        }
        int64_t want = 0;
        for (size_t a = 0; a < d; a++) want += (*coef)[a] * x[a];
        if (!at(x, &o) || o != want) return false;
    }
    return true;
}

// ── the kernel body ─────────────────────────────────────────────────────────────────────────────
struct Axis {
    std::string name;
    int64_t range = 1;   // guard bound, or the binding for a symbolic axis
    bool sym = false;
};

struct Kernel {
    std::vector<std::string> btype;      // element type of each binding ("f32", "f16", "i32", ...)
    bool params = false;                 // a params_n uniform is bound
    std::vector<Axis> axes;              // GIDVar axes in order of appearance
    int nloops = 0;
    std::string kv;                      // the loop variable (one loop)
    int64_t K = 0;
    bool ksym = false;
    std::string acc;
    int accop = 0;                       // '+' or 'M' (max)
    std::string acc_init;
    P upd, val, sidx;                    // the accumulator update operand, stored value, store index
};

// Parses the rendered module at symbolic binding n0; false for anything outside the single-reduce shape.
bool parse_kernel(const std::string &src, int64_t n0, Kernel *k) {
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
    size_t i = 0;
    for (; i < L.size() && !starts(L[i], "@compute"); i++) {
        const std::string &l = L[i];
        if (starts(l, "enable ") || starts(l, "struct ParamsN")) continue;
        if (!starts(l, "@group(0) @binding(")) return false;
        if (l.find("var<uniform> params_n") != std::string::npos) { k->params = true; continue; }
        char want[48];
        snprintf(want, sizeof want, "var<storage, %s> data%zu: array<", k->btype.empty() ? "read_write" : "read", k->btype.size());
        const size_t w = l.find(want);
        if (w == std::string::npos || l.size() < 3 || l.compare(l.size() - 2, 2, ">;") != 0) return false;
        const size_t t0 = w + strlen(want);
        k->btype.push_back(l.substr(t0, l.size() - 2 - t0));
    }
    if (k->btype.empty() || i == L.size()) return false;
    for (; i < L.size() && !starts(L[i], "let gid_x ="); i++)
        if (L[i].find("var<workgroup>") != std::string::npos) return false;
    if (i == L.size()) return false;
    i++;
    std::map<std::string, P> lets;
    int depth = 0, phase = 0;   // 0 before the accumulator, 1 in the loop, 2 after it
    bool stored = false;
    for (; i < L.size(); i++) {
        const std::string &l = L[i];
        if (l == "}") {
            if (depth == 0) { i++; break; }
            depth--;
            if (depth == 0) phase = 2;
            continue;
        }
        if (stored) return false;
        if (starts(l, "let ")) {
            const size_t c = l.find(':'), e = l.find('=');
            if (c == std::string::npos || e == std::string::npos || e < c || l.back() != ';') return false;
            const std::string name = trim(l.substr(4, c - 4)), rhs = trim(l.substr(e + 1, l.size() - e - 2));
            if (phase == 0 && rhs.find("flat_") != std::string::npos) {   // a GIDVar axis
                Axis ax{name, 1, false};
                long long r = 0, st = 0;
                char comp = 0, tail[8] = {0};
                if (sscanf(rhs.c_str(), "i32(flat_gid_%c %% %lldu)%7s", &comp, &r, tail) == 2 ||
                    sscanf(rhs.c_str(), "i32((flat_gid_%c / %lldu) %% %lldu)%7s", &comp, &st, &r, tail) == 3) {
                    ax.range = r;
                } else if (k->params && (sscanf(rhs.c_str(), "i32(flat_gid_%c)%7s", &comp, tail) == 1 ||
                                         sscanf(rhs.c_str(), "i32(flat_gid_%c / %lldu)%7s", &comp, &st, tail) == 2)) {
                    ax.sym = true;
                    ax.range = n0;
                } else {
                    return false;
                }
                if (comp != 'x' && comp != 'y' && comp != 'z') return false;
                k->axes.push_back(ax);
                continue;
            }
            P t;
            if (!parse_expr(rhs, lets, &t)) return false;
            lets[name] = t;
            continue;
        }
        if (starts(l, "if (")) {
            // axis guards and the symbolic bounds check; the guard bound must be the axis's range
            char name[32];
            long long r = 0;
            if (sscanf(l.c_str(), "if (%31[^ ] >= %lld) { return; }", name, &r) == 2) {
                bool found = false;
                for (auto &a : k->axes)
                    if (a.name == name && !a.sym && a.range == r) found = true;
                if (!found) return false;
                continue;
            }
            if (k->params && starts(l, "if (gid_x >= params_n.n0") && l.size() > 12 &&
                l.compare(l.size() - 11, 11, "{ return; }") == 0)
                continue;
            return false;
        }
        if (starts(l, "var ")) {
            if (phase != 0 || !k->acc.empty()) return false;
            const size_t c = l.find(':'), e = l.find('=');
            if (c == std::string::npos || e == std::string::npos || l.back() != ';') return false;
            k->acc = trim(l.substr(4, c - 4));
            if (trim(l.substr(c + 1, e - c - 1)) != "f32") return false;
            lets[k->acc] = mk(Node::VAR, "acc");   // read after the loop (the store and its lets)
            k->acc_init = trim(l.substr(e + 1, l.size() - e - 2));
            continue;
        }
        if (starts(l, "for (")) {
            if (phase != 0 || k->acc.empty() || depth != 0) return false;
            char a[32], b[32], c[32], bound[48];
            if (sscanf(l.c_str(), "for (var %31[^:]: i32 = 0; %31s < %47[^;]; %31[^+]++) {", a, b, bound, c) != 4) return false;
            if (std::string(a) != b || std::string(a) != c) return false;
            k->kv = a;
            const std::string bs = trim(bound);
            if (bs == "i32(params_n.n0)" && k->params) {
                k->ksym = true;
                k->K = n0;
            } else {
                char *end = nullptr;
                k->K = strtoll(bs.c_str(), &end, 10);
                if (!end || *end || k->K < 1) return false;
            }
            k->nloops++;
            depth = 1;
            phase = 1;
            continue;
        }
        if (phase == 1 && starts(l, (k->acc + " = ").c_str())) {
            if (k->upd) return false;
            const std::string rhs = trim(l.substr(k->acc.size() + 3, l.size() - k->acc.size() - 4));
            const std::string plus = k->acc + " + ";
            const std::string maxp = "max(" + k->acc + ", ";
            std::string e;
            if (starts(rhs, plus.c_str())) { k->accop = '+'; e = rhs.substr(plus.size()); }
            else if (starts(rhs, maxp.c_str()) && rhs.back() == ')') { k->accop = 'M'; e = rhs.substr(maxp.size(), rhs.size() - maxp.size() - 1); }
            else return false;
            if (!parse_expr(e, lets, &k->upd)) return false;
            continue;
        }
        if (phase == 2 && starts(l, "data0[") && l.back() == ';') {
            // data0[IDX] = VALUE;  (the index has balanced brackets)
            int d = 0;
            size_t j = 5;
            for (; j < l.size(); j++) {
                if (l[j] == '[') d++;
                else if (l[j] == ']' && --d == 0) break;
            }
            if (j >= l.size()) return false;
            const std::string idx = l.substr(6, j - 6), rest = trim(l.substr(j + 1));
            if (rest.size() < 3 || rest[0] != '=') return false;
            if (!parse_expr(idx, lets, &k->sidx) || !parse_expr(trim(rest.substr(1, rest.size() - 2)), lets, &k->val)) return false;
            stored = true;
            continue;
        }
        return false;
    }
    if (!stored || k->nloops != 1 || !k->upd || depth != 0 || i != L.size()) return false;
    // the accumulator may only appear through the store value: not in the loop's operand tree
    return true;
}

bool is_zero(const P &n) { return n->k == Node::NUM && n->num == 0.0; }
bool is_acc(const P &n) { return n->k == Node::VAR && n->s == "acc"; }

// A contraction operand: load, widened f16 load, ReLU prologue or mask prologue.
struct Operand {
    int buf = -1, zbuf = -1;
    P idx, zidx;
    int pro = 0;       // 0 none, 1 relu, 2 mask
    bool widened = false, zwidened = false;
};

P unwiden(const P &n, bool *w) {
    if (n->k == Node::CALL && n->s == "f32" && n->a.size() == 1 && n->a[0]->k == Node::LOAD) {
        *w = true;
        return n->a[0];
    }
    return n;
}

bool operand(const P &x0, Operand *o) {
    bool w = false;
    P x = unwiden(x0, &w);
    if (x->k == Node::LOAD) {
        o->buf = x->buf; o->idx = x->a[0]; o->widened = w;
        return true;
    }
    if (x->k == Node::CALL && x->s == "max" && x->a.size() == 2) {
        P a = x->a[0], b = x->a[1];
        if (is_zero(a)) std::swap(a, b);
        bool w2 = false;
        a = unwiden(a, &w2);
        if (a->k != Node::LOAD || !is_zero(b)) return false;
        o->buf = a->buf; o->idx = a->a[0]; o->widened = w2; o->pro = 1;
        return true;
    }
    if (x->k == Node::CALL && x->s == "select" && x->a.size() == 3 && is_zero(x->a[0])) {
        bool w2 = false;
        P adj = unwiden(x->a[1], &w2), c = x->a[2];
        if (adj->k != Node::LOAD || c->k != Node::BIN || c->s != "==") return false;
        P z = c->a[0], m = c->a[1];
        if (z->k == Node::CALL && z->s == "max") std::swap(z, m);
        bool w3 = false, w4 = false;
        z = unwiden(z, &w3);
        if (z->k != Node::LOAD || m->k != Node::CALL || m->s != "max" || m->a.size() != 2) return false;
        P mz = m->a[0], m0 = m->a[1];
        if (is_zero(mz)) std::swap(mz, m0);
        mz = unwiden(mz, &w4);
        if (!is_zero(m0) || !same(mz, z)) return false;
        o->buf = adj->buf; o->idx = adj->a[0]; o->widened = w2;
        o->zbuf = z->buf; o->zidx = z->a[0]; o->pro = 2; o->zwidened = w3 && w4;
        return true;
    }
    return false;
}

std::string dim(int64_t v, bool sym) { return sym ? std::string("sym") : std::to_string((long long)v); }

std::string fmt_float(double v) {
    char b[48];
    snprintf(b, sizeof b, "%a", (double)(float)v);   // exact f32 value, read back by strtof
    return b;
}

// One analysis at binding n0; "" when the kernel is not one of the template families.
std::string classify(const std::string &src, int64_t n0) {
    Kernel k;
    if (!parse_kernel(src, n0, &k)) return "";
    const int nb = (int)k.btype.size();
    // live output axes (guarded ranges > 1, or symbolic)
    std::vector<const Axis *> live;
    for (const Axis &a : k.axes)
        if (a.range > 1 || a.sym) live.push_back(&a);
    for (const Axis &a : k.axes)
        if (a.name == k.kv) return "";
    std::vector<std::string> vn;
    std::vector<int64_t> rg;
    std::vector<bool> sym;
    for (const Axis *a : live) { vn.push_back(a->name); rg.push_back(a->range); sym.push_back(a->sym); }
    vn.push_back(k.kv);
    rg.push_back(k.K);
    sym.push_back(k.ksym);
    for (const Axis &a : k.axes)   // one-point axes: indexes may name them (value 0)
        if (!(a.range > 1 || a.sym)) { vn.push_back(a.name); rg.push_back(1); sym.push_back(false); }
    const size_t kpos = live.size();
    for (int64_t r : rg)
        if (r > (1 << 16) || r < 1) return "";
    std::vector<int64_t> cs;
    if (!affine(k.sidx, vn, rg, &cs) || cs[kpos] != 0) return "";
    const std::string &out_t = k.btype[0];

    // ── plain reduction over one axis ──
    if (live.size() <= 1) {
        // the reduced value: a load (f16 widened), or the ReLU-backward mask of one (column sums)
        Operand o;
        if (!operand(k.upd, &o) || o.pro == 1) return "";
        const bool masked = o.pro == 2;
        if (o.buf < 1 || o.buf >= nb || nb != (masked ? 3 : 2) || out_t != "f32") return "";
        const std::string in_t = k.btype[o.buf];
        if ((in_t != "f32" && in_t != "f16") || o.widened != (in_t == "f16")) return "";
        std::string z_t;
        if (masked) {
            if (o.zbuf < 1 || o.zbuf >= nb || o.zbuf == o.buf || k.accop != '+') return "";
            z_t = k.btype[o.zbuf];
            if ((z_t != "f32" && z_t != "f16") || o.zwidened != (z_t == "f16")) return "";
        }
        float scale = 1.0f;
        P v = k.val;
        if (v->k == Node::BIN && v->s == "*") {
            P a = v->a[0], b = v->a[1];
            if (a->k == Node::NUM) std::swap(a, b);
            if (!is_acc(a) || b->k != Node::NUM) return "";
            scale = (float)b->num;
        } else if (!is_acc(v)) {
            return "";
        }
        if (k.accop == '+' && k.acc_init != "0.0") return "";
        if (k.accop == 'M' && (k.acc_init != "bitcast<f32>(0xff7fffffu)" || scale != 1.0f)) return "";
        std::vector<int64_t> ci;
        if (!affine(o.idx, vn, rg, &ci)) return "";
        if (masked) {   // the mask reads Z at A's element
            std::vector<int64_t> cz;
            if (!affine(o.zidx, vn, rg, &cz) || cz != ci) return "";
        }
        std::string M, N;
        int axis;
        if (live.empty()) {   // out[0] = reduce over k of in[k]
            if (ci[0] != 1) return "";
            axis = 1; M = "1"; N = dim(k.K, k.ksym);
        } else if (cs[0] != 1) {
            return "";
        } else if (ci[1] == 1 && ci[0] == k.K) {   // in[o, k]: across a row
            axis = 1; M = dim(rg[0], sym[0]); N = dim(k.K, k.ksym);
        } else if (ci[0] == 1 && ci[1] == rg[0]) { // in[k, o]: down a column
            axis = 0; M = dim(k.K, k.ksym); N = dim(rg[0], sym[0]);
        } else {
            return "";
        }
        if (masked && axis != 0) return "";
        std::string key = "tmpl:reduce;op=" + std::string(k.accop == '+' ? "sum" : "max") + ";axis=" + std::to_string(axis) +
                          ";M=" + M + ";N=" + N;
        if (in_t == "f16") key += ";dtype=f16";
        if (scale != 1.0f) key += ";scale=" + fmt_float(scale);
        if (masked)
            key += ";pa=mask;in_a=" + std::to_string(o.buf) + ";za=" + std::to_string(o.zbuf) + (z_t == "f16" ? ";wza=1" : "");
        return key;
    }

    // ── contraction ──
    if (live.size() != 2 || k.accop != '+' || k.acc_init != "0.0") return "";
    if (k.upd->k != Node::BIN || k.upd->s != "*") return "";
    Operand op[2];
    if (!operand(k.upd->a[0], &op[0]) || !operand(k.upd->a[1], &op[1])) return "";
    // C = cm*m + n (row-major [M,N]): which live axis is m
    int im, in;
    if (cs[1] == 1 && cs[0] == rg[1]) { im = 0; in = 1; }
    else if (cs[0] == 1 && cs[1] == rg[0]) { im = 1; in = 0; }
    else return "";
    const int64_t M = rg[im], N = rg[in], K = k.K;
    std::vector<int64_t> c0, c1;
    if (!affine(op[0].idx, vn, rg, &c0) || !affine(op[1].idx, vn, rg, &c1)) return "";
    int ia = -1;
    if (c0[in] == 0 && (c0[im] != 0 || M == 1)) ia = 0;
    else if (c1[in] == 0 && (c1[im] != 0 || M == 1)) ia = 1;
    if (ia < 0) return "";
    const Operand &A = op[ia], &B = op[1 - ia];
    const std::vector<int64_t> &ca = ia == 0 ? c0 : c1, &cb = ia == 0 ? c1 : c0;
    if (cb[im] != 0) return "";
    int ta, tb;
    if (ca[2] == 1 && ca[im] == K) ta = 0;
    else if (ca[im] == 1 && ca[2] == M) ta = 1;
    else return "";
    if (cb[2] == 1 && cb[in] == K) tb = 0;
    else if (cb[in] == 1 && cb[2] == N) tb = 1;
    else return "";
    // a mask source is read at the operand's own index
    for (const Operand *o : {&A, &B})
        if (o->pro == 2) {
            std::vector<int64_t> cz, cd;
            if (!affine(o->zidx, vn, rg, &cz) || !affine(o->idx, vn, rg, &cd) || cz != cd) return "";
        }
    // operand dtypes: all f16 widened in the loop (an f16 reduce, codegen/lower.go:667-716), or an f32
    // contraction whose f16 operands (and mask sources) are widened in the loop (an f32 adjoint times an
    // f16 weight or activation, the promotion of tensor/ops.go:74-79): those get the wa/wb/wza/wzb flags
    bool any32 = false;
    for (const Operand *o : {&A, &B}) {
        const int bufs[2] = {o->buf, o->zbuf};
        for (int b : bufs) {
            if (b < 0) continue;
            if (b < 1 || b >= nb) return "";
            const std::string &t = k.btype[b];
            if (t != "f32" && t != "f16") return "";
            any32 |= t == "f32";
        }
    }
    const std::string dt = any32 ? "f32" : "f16";
    bool wflag[2] = {false, false}, wzflag[2] = {false, false};
    for (int r = 0; r < 2; r++) {
        const Operand *o = r == 0 ? &A : &B;
        const bool f16buf = k.btype[o->buf] == "f16";
        if (o->widened != f16buf) return "";   // an f16 load is widened, an f32 one is not
        wflag[r] = any32 && f16buf;
        if (o->zbuf >= 0) {
            const bool f16z = k.btype[o->zbuf] == "f16";
            if (o->zwidened != f16z) return "";
            wzflag[r] = any32 && f16z;
        }
    }
    // epilogue
    std::string epi = "store";
    float scale = 1.0f;
    int bias = -1;
    P v = k.val;
    auto accv = [&](const P &x) {
        if (dt == "f16") return x->k == Node::CALL && x->s == "f16" && x->a.size() == 1 && is_acc(x->a[0]);
        return is_acc(x);
    };
    auto bias_sum = [&](const P &x) -> bool {
        if (x->k != Node::BIN || x->s != "+") return false;
        P a = x->a[0], b = x->a[1];
        if (!accv(a)) std::swap(a, b);
        if (!accv(a) || b->k != Node::LOAD) return false;
        std::vector<int64_t> cbias;
        if (!affine(b->a[0], vn, rg, &cbias) || cbias[in] != 1 || cbias[im] != 0 || cbias[2] != 0) return false;
        bias = b->buf;
        return true;
    };
    if (accv(v)) {
        epi = "store";
    } else if (dt == "f32" && v->k == Node::BIN && v->s == "*" &&
               ((is_acc(v->a[0]) && v->a[1]->k == Node::NUM) || (is_acc(v->a[1]) && v->a[0]->k == Node::NUM))) {
        scale = (float)(v->a[0]->k == Node::NUM ? v->a[0]->num : v->a[1]->num);
    } else if (bias_sum(v)) {
        epi = "bias";
    } else if (v->k == Node::CALL && v->s == "max" && v->a.size() == 2 &&
               (is_zero(v->a[1]) || is_zero(v->a[0])) && bias_sum(is_zero(v->a[1]) ? v->a[0] : v->a[1])) {
        epi = "bias_relu";   // f16: max(f16(acc) + bias, 0), the f16 add rounding once as the template's does
    } else {
        return "";
    }
    if (out_t != dt) return "";
    if (bias >= 0 && (bias < 1 || bias >= nb || k.btype[bias] != dt)) return "";
    // every input binding is used exactly once in its role
    std::vector<int> roles = {A.buf, B.buf};
    if (A.zbuf >= 0) roles.push_back(A.zbuf);
    if (B.zbuf >= 0) roles.push_back(B.zbuf);
    if (bias >= 0) roles.push_back(bias);
    if ((int)roles.size() != nb - 1) return "";
    for (size_t x = 0; x < roles.size(); x++)
        for (size_t y = x + 1; y < roles.size(); y++)
            if (roles[x] == roles[y]) return "";
    const std::string Ms = dim(M, sym[im]), Ns = dim(N, sym[in]), Ks = dim(K, k.ksym);
    std::string key = "tmpl:gemm;dtype=" + dt + ";epi=" + epi + ";ta=" + std::to_string(ta) + ";tb=" + std::to_string(tb) +
                      ";M=" + Ms + ";N=" + Ns + ";K=" + Ks;
    if (scale != 1.0f) key += ";scale=" + fmt_float(scale);
    static const char *pro[] = {"", "relu", "mask"};
    if (A.pro) key += std::string(";pa=") + pro[A.pro];
    if (B.pro) key += std::string(";pb=") + pro[B.pro];
    if (wflag[0]) key += ";wa=1";
    if (wflag[1]) key += ";wb=1";
    if (wzflag[0]) key += ";wza=1";
    if (wzflag[1]) key += ";wzb=1";
    // PARAM roles: the default order (A, B, bias) or the two operands swapped is written as before
    // (swap_ab=1); any other order names each role's PARAM
    const bool plain = A.zbuf < 0 && B.zbuf < 0 && (bias < 0 || bias == 3);
    if (plain && A.buf == 1 && B.buf == 2) {
    } else if (plain && A.buf == 2 && B.buf == 1) {
        key += ";swap_ab=1";
    } else {
        key += ";in_a=" + std::to_string(A.buf) + ";in_b=" + std::to_string(B.buf);
        if (bias >= 0) key += ";in_bias=" + std::to_string(bias);
        if (A.zbuf >= 0) key += ";za=" + std::to_string(A.zbuf);
        if (B.zbuf >= 0) key += ";zb=" + std::to_string(B.zbuf);
    }
    return key;
}

}  // namespace

bool wgsl_match_contraction(const std::string &src, std::string *key) {
    // a symbolic kernel is analysed at two bindings; its symbolic ranges print as "sym", so the two
    // keys agree only when no coefficient depends on the binding
    const std::string a = classify(src, 37);
    if (a.empty()) return false;
    if (src.find("params_n") != std::string::npos && classify(src, 64) != a) return false;
    *key = a;
    return true;
}

}  // namespace ah
