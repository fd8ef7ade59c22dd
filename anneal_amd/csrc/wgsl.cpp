// wgsl.cpp — renders the WGSL that anneal's codegen emits as HIP C++ for hiprtc (gfx950).
//
// The reference's schedule cache pre-renders every kernel and keeps only the source string
// (schedule/cache.go:69-100), so a backend that takes its ExecItems unchanged has to work from that
// string. codegen/wgsl.go:41-238 emits a small, line-oriented subset of WGSL:
//   module scope: `enable f16;`, storage bindings `@group(0) @binding(i) var<storage, A> NAME: array<T>;`,
//     the symbolic uniform `struct ParamsN {...}` + `var<uniform> params_n: ParamsN;`,
//     `@compute @workgroup_size(x, y, z)`, workgroup arrays `var<workgroup> NAME: array<T, N>;`,
//     `fn main(@builtin(global_invocation_id) gid, @builtin(workgroup_id) wid, @builtin(local_invocation_id) lid) {`;
//   body: one statement per line — `let`/`var` declarations, `for (var rN: i32 = 0; ...; rN++) {`,
//     `if (...) {` / `if (...) { return; }`, `}`, `workgroupBarrier();`, assignments and stores;
//   expressions: the ALU renderings of codegen/wgsl.go:253-312 (`select`, `exp2`, `log2`, `sin`,
//     `sqrt`, `trunc`, `max`, `pow`, casts `T(x)`, `bitcast<T>(x)`), literals of constLiteral
//     (:314-352), and `vec4<f32>(...)` from the vectorized Opt path (codegen/lower.go:865-941).
// Each line is rewritten independently: declarations get C++ types, WGSL calls become calls to the
// helpers of the prelude below (overloaded per element type, so no type inference is needed), and
// unsuffixed float literals get an `f` suffix so arithmetic stays in f32 as in WGSL. Anything outside
// the subset is rejected with a message rather than guessed.
#include <ctype.h>
#include <string.h>

#include <string>
#include <vector>

#include "ah_internal.h"

namespace ah {

namespace {

const char *kPrelude = R"HIP(
typedef _Float16 wg_f16;
struct wg_uvec3 { unsigned x, y, z; };
__device__ __forceinline__ float wg_exp2(float x) { return exp2f(x); }
__device__ __forceinline__ wg_f16 wg_exp2(wg_f16 x) { return (wg_f16)exp2f((float)x); }
__device__ __forceinline__ float wg_log2(float x) { return log2f(x); }
__device__ __forceinline__ wg_f16 wg_log2(wg_f16 x) { return (wg_f16)log2f((float)x); }
__device__ __forceinline__ float wg_sin(float x) { return sinf(x); }
__device__ __forceinline__ wg_f16 wg_sin(wg_f16 x) { return (wg_f16)sinf((float)x); }
__device__ __forceinline__ float wg_sqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ wg_f16 wg_sqrt(wg_f16 x) { return (wg_f16)sqrtf((float)x); }
__device__ __forceinline__ float wg_trunc(float x) { return truncf(x); }
__device__ __forceinline__ wg_f16 wg_trunc(wg_f16 x) { return (wg_f16)truncf((float)x); }
__device__ __forceinline__ float wg_pow(float x, float y) { return powf(x, y); }
__device__ __forceinline__ wg_f16 wg_pow(wg_f16 x, wg_f16 y) { return (wg_f16)powf((float)x, (float)y); }
__device__ __forceinline__ float wg_max(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ wg_f16 wg_max(wg_f16 a, wg_f16 b) { return a > b ? a : (b > a ? b : (a == a ? a : b)); }
__device__ __forceinline__ int wg_max(int a, int b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned wg_max(unsigned a, unsigned b) { return a > b ? a : b; }
__device__ __forceinline__ float wg_min(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ int wg_min(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ unsigned wg_min(unsigned a, unsigned b) { return a < b ? a : b; }
__device__ __forceinline__ float wg_abs(float a) { return fabsf(a); }
__device__ __forceinline__ int wg_abs(int a) { return a < 0 ? -a : a; }
// WGSL float->integer conversions round toward zero and saturate (no undefined cases)
template <class To, class From> __device__ __forceinline__ To wg_cvt(From v) { return (To)v; }
template <> __device__ __forceinline__ int wg_cvt<int, float>(float v) {
    return v != v ? 0 : v >= 2147483520.0f ? 2147483647 : v <= -2147483648.0f ? (-2147483647 - 1) : (int)v;
}
template <> __device__ __forceinline__ unsigned wg_cvt<unsigned, float>(float v) {
    return v != v || v <= 0.0f ? 0u : v >= 4294967040.0f ? 4294967295u : (unsigned)v;
}
template <> __device__ __forceinline__ int wg_cvt<int, wg_f16>(wg_f16 v) { return wg_cvt<int, float>((float)v); }
template <> __device__ __forceinline__ unsigned wg_cvt<unsigned, wg_f16>(wg_f16 v) { return wg_cvt<unsigned, float>((float)v); }
template <class To, class From> __device__ __forceinline__ To wg_bitcast(From v) {
    if constexpr (sizeof(To) == sizeof(From)) return __builtin_bit_cast(To, v);
    else if constexpr (sizeof(To) == 2) return __builtin_bit_cast(To, (unsigned short)v);
    else return __builtin_bit_cast(To, (unsigned)__builtin_bit_cast(unsigned short, v));
}
__device__ __forceinline__ float wg_wave_sum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wg_wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
struct wg_vec4 { float x, y, z, w; };
__device__ __forceinline__ wg_vec4 wg_make4(float a, float b, float c, float d) { return wg_vec4{a, b, c, d}; }
__device__ __forceinline__ wg_vec4 wg_make4(float a) { return wg_vec4{a, a, a, a}; }
__device__ __forceinline__ wg_vec4 operator+(wg_vec4 a, wg_vec4 b) { return {a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w}; }
__device__ __forceinline__ wg_vec4 operator*(wg_vec4 a, wg_vec4 b) { return {a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w}; }
__device__ __forceinline__ wg_vec4 operator*(float a, wg_vec4 b) { return {a * b.x, a * b.y, a * b.z, a * b.w}; }
__device__ __forceinline__ wg_vec4 operator*(wg_vec4 a, float b) { return {a.x * b, a.y * b, a.z * b, a.w * b}; }
)HIP";

struct Tok {
    std::string s;
    bool ident = false, number = false;
};

bool is_ident_start(char c) { return isalpha((unsigned char)c) || c == '_'; }
bool is_ident_char(char c) { return isalnum((unsigned char)c) || c == '_'; }

// Splits an expression into identifiers, numbers and single/double-character operators.
bool tokenize(const std::string &e, std::vector<Tok> &out, std::string *err) {
    size_t i = 0;
    while (i < e.size()) {
        char c = e[i];
        if (isspace((unsigned char)c)) { i++; continue; }
        Tok t;
        if (is_ident_start(c)) {
            size_t j = i;
            while (j < e.size() && is_ident_char(e[j])) j++;
            t.s = e.substr(i, j - i);
            t.ident = true;
            i = j;
        } else if (isdigit((unsigned char)c) || (c == '.' && i + 1 < e.size() && isdigit((unsigned char)e[i + 1]))) {
            size_t j = i;
            if (c == '0' && j + 1 < e.size() && (e[j + 1] == 'x' || e[j + 1] == 'X')) {
                j += 2;
                while (j < e.size() && isxdigit((unsigned char)e[j])) j++;
            } else {
                while (j < e.size() && (isdigit((unsigned char)e[j]) || e[j] == '.')) j++;
                if (j < e.size() && (e[j] == 'e' || e[j] == 'E')) {
                    j++;
                    if (j < e.size() && (e[j] == '+' || e[j] == '-')) j++;
                    while (j < e.size() && isdigit((unsigned char)e[j])) j++;
                }
            }
            if (j < e.size() && (e[j] == 'u' || e[j] == 'i' || e[j] == 'f' || e[j] == 'h')) j++;
            t.s = e.substr(i, j - i);
            t.number = true;
            i = j;
        } else {
            static const char *two[] = {"<=", ">=", "==", "!=", "&&", "||", "<<", ">>", "++", "--"};
            bool matched = false;
            for (const char *op : two)
                if (e.compare(i, 2, op) == 0) { t.s = op; i += 2; matched = true; break; }
            if (!matched) {
                if (!strchr("+-*/%<>=!&|^~()[],.?:", c)) {
                    *err = std::string("unexpected character '") + c + "' in expression: " + e;
                    return false;
                }
                t.s = std::string(1, c);
                i++;
            }
        }
        out.push_back(t);
    }
    return true;
}

// WGSL scalar / vector type name -> C++ type, or "" if unknown.
std::string ctype(const std::string &t) {
    if (t == "f32") return "float";
    if (t == "f16") return "wg_f16";
    if (t == "i32") return "int";
    if (t == "u32") return "unsigned";
    if (t == "bool") return "bool";
    if (t == "vec4<f32>") return "wg_vec4";
    return "";
}

std::string number(const std::string &n) {
    const char last = n.back();
    const bool hex = n.size() > 1 && (n[1] == 'x' || n[1] == 'X');
    if (hex) return n;                                              // 0x...u stays unsigned
    if (last == 'u') return n;
    if (last == 'i') return n.substr(0, n.size() - 1);
    if (last == 'h') return "((wg_f16)" + n.substr(0, n.size() - 1) + "f)";
    const bool is_float = n.find('.') != std::string::npos || n.find('e') != std::string::npos ||
                          n.find('E') != std::string::npos;
    if (last == 'f') return is_float ? n : n.substr(0, n.size() - 1) + ".0f";
    return is_float ? n + "f" : n;
}

struct ExprRenderer {
    const std::vector<Tok> &t;
    size_t p = 0;
    std::string *err;
    ExprRenderer(const std::vector<Tok> &tt, std::string *e) : t(tt), err(e) {}

    // Renders tokens until an unmatched ')' or top-level ',' (not consumed) or the end.
    bool seq(std::string &out) {
        int depth = 0;
        while (p < t.size()) {
            const Tok &k = t[p];
            if (k.s == ")" && depth == 0) return true;
            if (k.s == "," && depth == 0) return true;
            if (k.s == "(" || k.s == "[") depth++;
            if ((k.s == ")" || k.s == "]") && depth > 0) depth--;
            if (k.ident && !rend_ident(out)) return false;
            if (!k.ident) {
                out += k.number ? number(k.s) : k.s;
                out += ' ';
                p++;
            }
        }
        return true;
    }

    bool args(std::vector<std::string> &a) {   // at '('; consumes through the matching ')'
        p++;
        if (p < t.size() && t[p].s == ")") { p++; return true; }
        while (true) {
            std::string one;
            if (!seq(one)) return false;
            a.push_back(one);
            if (p >= t.size()) { *err = "unbalanced parentheses"; return false; }
            if (t[p].s == ",") { p++; continue; }
            p++;   // ')'
            return true;
        }
    }

    bool rend_ident(std::string &out) {
        std::string name = t[p].s;
        p++;
        std::string targ;   // template argument of bitcast<T> / vec4<T>
        if ((name == "bitcast" || name == "vec4" || name == "vec3" || name == "vec2") && p < t.size() && t[p].s == "<") {
            size_t q = p + 1;
            while (q < t.size() && t[q].s != ">") targ += t[q++].s;
            if (q >= t.size()) { *err = "unterminated template argument after " + name; return false; }
            p = q + 1;
        }
        if (p >= t.size() || t[p].s != "(") {   // variable, builtin or member access
            if (name == "true" || name == "false") out += name + " ";
            else out += name + " ";
            return true;
        }
        std::vector<std::string> a;
        if (!args(a)) return false;
        auto need = [&](size_t n) {
            if (a.size() != n) { *err = name + "() takes " + std::to_string(n) + " arguments"; return false; }
            return true;
        };
        if (name == "select") {
            if (!need(3)) return false;
            out += "((" + a[2] + ") ? (" + a[1] + ") : (" + a[0] + ")) ";
        } else if (name == "bitcast") {
            const std::string ct = ctype(targ);
            if (ct.empty() || !need(1)) { if (ct.empty()) *err = "bitcast to " + targ; return false; }
            out += "wg_bitcast<" + ct + ">(" + a[0] + ") ";
        } else if (name == "vec4") {
            if (targ != "f32" || (a.size() != 1 && a.size() != 4)) { *err = "vec4<" + targ + "> constructor"; return false; }
            out += "wg_make4(";
            for (size_t i = 0; i < a.size(); i++) out += (i ? ", " : "") + a[i];
            out += ") ";
        } else if (!ctype(name).empty()) {   // conversion T(x)
            if (!need(1)) return false;
            out += "wg_cvt<" + ctype(name) + ">(" + a[0] + ") ";
        } else if (name == "exp2" || name == "log2" || name == "sin" || name == "sqrt" || name == "trunc" ||
                   name == "abs") {
            if (!need(1)) return false;
            out += "wg_" + name + "(" + a[0] + ") ";
        } else if (name == "max" || name == "min" || name == "pow") {
            if (!need(2)) return false;
            out += "wg_" + name + "(" + a[0] + ", " + a[1] + ") ";
        } else {
            *err = "unsupported WGSL function " + name;
            return false;
        }
        return true;
    }
};

bool expr(const std::string &e, std::string &out, std::string *err) {
    std::vector<Tok> toks;
    if (!tokenize(e, toks, err)) return false;
    ExprRenderer r(toks, err);
    if (!r.seq(out)) return false;
    if (r.p != toks.size()) { *err = "unbalanced ')' in expression: " + e; return false; }
    return true;
}

std::string trim(const std::string &s) {
    size_t a = 0, b = s.size();
    while (a < b && isspace((unsigned char)s[a])) a++;
    while (b > a && isspace((unsigned char)s[b - 1])) b--;
    return s.substr(a, b - a);
}

bool starts(const std::string &s, const char *p) { return s.compare(0, strlen(p), p) == 0; }

// "NAME: T = EXPR" or "NAME = EXPR" (after let/var) -> C++ declaration.
bool decl(const std::string &rest, bool is_const, std::string &out, std::string *err) {
    size_t eq = rest.find('=');
    if (eq == std::string::npos) { *err = "declaration without initializer: " + rest; return false; }
    std::string lhs = trim(rest.substr(0, eq)), rhs = trim(rest.substr(eq + 1));
    if (!rhs.empty() && rhs.back() == ';') rhs.pop_back();
    std::string name = lhs, ty = "auto";
    size_t colon = lhs.find(':');
    if (colon != std::string::npos) {
        name = trim(lhs.substr(0, colon));
        std::string wt = trim(lhs.substr(colon + 1));
        ty = ctype(wt);
        if (ty.empty()) { *err = "unsupported type " + wt; return false; }
    }
    std::string r;
    if (!expr(rhs, r, err)) return false;
    out = std::string(is_const ? "const " : "") + ty + " " + name + " = (" + ty + ")(" + r + ");";
    if (ty == "auto") out = std::string(is_const ? "const " : "") + "auto " + name + " = " + r + ";";
    return true;
}

}  // namespace

// Wave-per-output form of a single-reduce kernel. codegen/lower.go:654-719 gives every output element
// one thread that runs the whole reduce loop serially. When the body is exactly: output-axis lets and
// guards, one f32 accumulator, one outermost loop (nested loops inside allowed) whose statements are lets
// and the accumulator's update `acc = acc + e` or `acc = max(acc, e)`, then lets and stores, the kernel
// is rendered with one 64-lane wave per output element instead: lane l runs the outermost loop's
// iterations l, l+64, ..., the lanes' partials are combined by a shuffle tree (sum or max), and lane 0
// runs the statements after the loop. Sums then add in a different (fixed) order than the serial loop.
// Returns the line indices (of `lines`) of the accumulator's declaration and of the outermost loop's
// first and closing lines, with the accumulator's name and update operator.
struct WavePlan {
    bool ok = false;
    size_t decl = 0, loop = 0, close = 0;
    std::string acc;
    bool is_max = false;
};

WavePlan plan_wave(const std::vector<std::string> &lines, size_t body_start) {
    WavePlan w;
    int depth = 0;
    bool in_loop = false, after = false, updated = false;
    for (size_t i = body_start; i < lines.size(); i++) {
        std::string l = trim(lines[i]);
        if (l.empty() || starts(l, "//")) continue;
        if (l == "}") {
            if (depth == 0) return (w.ok = after && updated, w);
            depth--;
            if (in_loop && depth == 0) { w.close = i; in_loop = false; after = true; }
            continue;
        }
        if (l.find("workgroupBarrier") != std::string::npos || l.find("lid.") != std::string::npos ||
            (l.find("wid.") != std::string::npos && !starts(l, "let flat_wid_")))
            return w;
        if (starts(l, "var ")) {
            if (!w.acc.empty() || in_loop || after) return w;
            const size_t c = l.find(':'), e = l.find('=');
            if (c == std::string::npos || e == std::string::npos || trim(l.substr(c + 1, e - c - 1)) != "f32") return w;
            w.acc = trim(l.substr(4, c - 4));
            w.decl = i;
            continue;
        }
        if (starts(l, "for (")) {
            if (w.acc.empty() || after) return w;
            if (!in_loop) { in_loop = true; w.loop = i; }
            depth++;
            continue;
        }
        if (starts(l, "if (")) {
            // only the early-return guards before the accumulator
            if (!w.acc.empty() || l.size() < 12 || l.compare(l.size() - 11, 11, "{ return; }") != 0) return w;
            continue;
        }
        if (starts(l, "let ")) continue;
        if (!w.acc.empty() && starts(l, (w.acc + " = ").c_str())) {
            if (!in_loop || updated) return w;
            const std::string r = trim(l.substr(w.acc.size() + 3));
            if (starts(r, (w.acc + " + ").c_str())) w.is_max = false;
            else if (starts(r, ("max(" + w.acc + ", ").c_str())) w.is_max = true;
            else return w;
            updated = true;
            continue;
        }
        if (after && starts(l, "data")) continue;   // stores after the loop
        return w;
    }
    return w;
}

// Returns HIP source with an extern "C" entry point `kernel`, or "" with *err set. *wave (optional) is set
// when the kernel was rendered in the wave-per-output form (launched with 64 lanes per original thread).
std::string wgsl_to_hip(const std::string &src, std::string *err, bool *wave) {
    std::vector<std::string> lines;
    {
        size_t a = 0;
        while (a <= src.size()) {
            size_t b = src.find('\n', a);
            if (b == std::string::npos) b = src.size();
            lines.push_back(src.substr(a, b - a));
            a = b + 1;
        }
    }
    struct Param { int binding; std::string decl; };
    std::vector<Param> params;
    std::vector<std::string> shared;
    bool symbolic = false;
    long ws[3] = {64, 1, 1};
    std::string body;
    int depth = 0;
    size_t i = 0;
    // module scope
    for (; i < lines.size(); i++) {
        std::string l = trim(lines[i]);
        if (l.empty() || starts(l, "//") || l == "enable f16;") continue;
        if (starts(l, "struct ParamsN")) continue;
        if (starts(l, "@group(")) {
            int binding = -1;
            if (sscanf(l.c_str(), "@group(0) @binding(%d)", &binding) != 1) { *err = "bad binding: " + l; return ""; }
            if (l.find("var<uniform>") != std::string::npos) {
                if (l.find("params_n") == std::string::npos) { *err = "unsupported uniform: " + l; return ""; }
                symbolic = true;
                continue;
            }
            size_t v = l.find("var<storage,"), gt = l.find('>', v), colon = l.find(':', gt);
            size_t arr = l.find("array<", colon), end = l.rfind('>');
            if (v == std::string::npos || gt == std::string::npos || colon == std::string::npos ||
                arr == std::string::npos || end == std::string::npos || end < arr) {
                *err = "unsupported binding: " + l;
                return "";
            }
            const std::string access = trim(l.substr(v + 12, gt - v - 12));
            const std::string name = trim(l.substr(gt + 1, colon - gt - 1));
            const std::string et = ctype(trim(l.substr(arr + 6, end - arr - 6)));
            if (et.empty()) { *err = "unsupported element type: " + l; return ""; }
            params.push_back({binding, std::string(access == "read" ? "const " : "") + et + " *__restrict__ " + name});
            continue;
        }
        if (starts(l, "@compute")) {
            size_t w = l.find("@workgroup_size(");
            if (w != std::string::npos) {
                long x = 1, y = 1, z = 1;
                int n = sscanf(l.c_str() + w, "@workgroup_size(%ld, %ld, %ld)", &x, &y, &z);
                if (n < 1) n = sscanf(l.c_str() + w, "@workgroup_size(%ld,%ld,%ld)", &x, &y, &z);
                if (n < 1) { *err = "bad workgroup_size: " + l; return ""; }
                ws[0] = x; ws[1] = n > 1 ? y : 1; ws[2] = n > 2 ? z : 1;
            }
            continue;
        }
        if (starts(l, "var<workgroup>")) {
            // var<workgroup> NAME: array<T, N>;
            size_t colon = l.find(':'), arr = l.find("array<"), comma = l.rfind(','), end = l.rfind('>');
            if (colon == std::string::npos || arr == std::string::npos || comma == std::string::npos || end == std::string::npos) {
                *err = "bad workgroup array: " + l;
                return "";
            }
            const std::string name = trim(l.substr(14, colon - 14));
            const std::string et = ctype(trim(l.substr(arr + 6, comma - arr - 6)));
            const std::string n = trim(l.substr(comma + 1, end - comma - 1));
            if (et.empty()) { *err = "unsupported workgroup element type: " + l; return ""; }
            shared.push_back("__shared__ " + et + " " + name + "[" + n + "];");
            continue;
        }
        if (starts(l, "fn main")) {
            // skip the builtin parameter list up to the opening brace
            while (i < lines.size() && lines[i].find('{') == std::string::npos) i++;
            i++;
            break;
        }
        *err = "unsupported module-scope line: " + l;
        return "";
    }
    // body
    WavePlan wp;
    if (wave) {
        wp = plan_wave(lines, i);
        *wave = wp.ok && shared.empty();
        wp.ok = *wave;
    }
    for (; i < lines.size(); i++) {
        std::string l = trim(lines[i]);
        if (l.empty() || starts(l, "//")) continue;
        std::string out;
        if (wp.ok && i == wp.loop) {
            // for (var rN: i32 = 0; COND; rN++) {  ->  the lane's strided share of the iterations
            char v[32];
            if (sscanf(l.c_str(), "for (var %31[^:]: i32 = 0;", v) != 1) { *err = "unsupported reduce loop: " + l; return ""; }
            const size_t s1 = l.find(';'), s2 = l.find(';', s1 + 1);
            std::string c;
            if (!expr(trim(l.substr(s1 + 1, s2 - s1 - 1)), c, err)) return "";
            out = std::string("for (int ") + v + " = (int)wg_lane; " + c + "; " + v + " += 64) {";
            depth++;
        } else if (wp.ok && i == wp.close) {
            depth--;
            out = "}\n" + std::string(2 * (depth + 1), ' ') + wp.acc + " = " + (wp.is_max ? "wg_wave_max(" : "wg_wave_sum(") +
                  wp.acc + ");\n" + std::string(2 * (depth + 1), ' ') + "if (wg_lane != 0u) return;";
        } else if (l == "}") {
            if (depth == 0) { depth = -1; break; }   // end of main
            out = "}";
            depth--;
        } else if (starts(l, "let ")) {
            if (!decl(l.substr(4), true, out, err)) return "";
        } else if (starts(l, "var ")) {
            if (!decl(l.substr(4), false, out, err)) return "";
        } else if (starts(l, "for (")) {
            // for (var rN: T = INIT; COND; STEP) {
            size_t s1 = l.find(';'), s2 = l.find(';', s1 + 1), close = l.rfind(')');
            if (s1 == std::string::npos || s2 == std::string::npos || close == std::string::npos || l.back() != '{') {
                *err = "unsupported for statement: " + l;
                return "";
            }
            std::string init = trim(l.substr(5, s1 - 5)), cond = trim(l.substr(s1 + 1, s2 - s1 - 1));
            std::string step = trim(l.substr(s2 + 1, close - s2 - 1));
            if (!starts(init, "var ")) { *err = "unsupported for initializer: " + l; return ""; }
            std::string d, c, st;
            if (!decl(init.substr(4), false, d, err) || !expr(cond, c, err) || !expr(step, st, err)) return "";
            d.pop_back();   // ';'
            out = "for (" + d + "; " + c + "; " + st + ") {";
            depth++;
        } else if (starts(l, "if (")) {
            size_t close = l.rfind(')');
            const bool ret = l.size() > 10 && l.compare(l.size() - 11, 11, "{ return; }") == 0;
            if (ret) close = l.rfind(')', l.size() - 11);
            if (close == std::string::npos || close < 4) { *err = "unsupported if: " + l; return ""; }
            std::string c;
            if (!expr(l.substr(4, close - 4), c, err)) return "";
            if (ret) out = "if (" + c + ") { return; }";
            else if (l.back() == '{') { out = "if (" + c + ") {"; depth++; }
            else { *err = "unsupported if: " + l; return ""; }
        } else if (l == "workgroupBarrier();") {
            out = "__syncthreads();";
        } else if (l == "return;") {
            out = "return;";
        } else {
            // assignment or store: LHS = EXPR;   (also `x += y;` style compound forms)
            if (l.back() != ';') { *err = "unsupported statement: " + l; return ""; }
            size_t eq = std::string::npos;
            for (size_t k = 0; k < l.size(); k++) {
                if (l[k] == '=' && (k + 1 >= l.size() || l[k + 1] != '=') && (k == 0 || !strchr("=!<>", l[k - 1]))) { eq = k; break; }
            }
            if (eq == std::string::npos) { *err = "unsupported statement: " + l; return ""; }
            std::string op = "=";
            size_t lend = eq;
            if (eq > 0 && strchr("+-*/", l[eq - 1])) { op = std::string(1, l[eq - 1]) + "="; lend = eq - 1; }
            std::string a, b;
            if (!expr(l.substr(0, lend), a, err) || !expr(l.substr(eq + 1, l.size() - eq - 2), b, err)) return "";
            out = a + op + " " + b + ";";
        }
        body += std::string(2 * (depth + 1), ' ') + out + "\n";
    }
    if (depth != -1) { *err = "unterminated fn main"; return ""; }
    // assemble
    std::string s = kPrelude;
    const long nthreads = wp.ok ? 64 : ws[0] * ws[1] * ws[2];
    s += "\nextern \"C\" __global__ void __launch_bounds__(" + std::to_string(nthreads) + ") kernel(";
    for (size_t k = 0; k < params.size(); k++) {
        if (params[k].binding != (int)k) { *err = "bindings must be 0..n-1 in order"; return ""; }
        s += (k ? ", " : "") + params[k].decl;
    }
    if (symbolic) s += std::string(params.empty() ? "" : ", ") + "int wg_n0, int wg_n1, int wg_n2, int wg_n3";
    s += ") {\n";
    for (auto &sh : shared) s += "  " + sh + "\n";
    if (wp.ok) {
        // one wave per original thread: the grid's blocks are the original threads (ah_launch scales it)
        s += "  // wave-per-output rendering: lane wg_lane of the wave that stands for one original thread\n";
        s += "  const unsigned wg_lane = threadIdx.x;\n";
        s += "  const wg_uvec3 gid = {blockIdx.x, blockIdx.y, blockIdx.z};\n";
        s += "  const wg_uvec3 wid = {0u, 0u, 0u};\n";
    } else {
        s += "  const wg_uvec3 lid = {threadIdx.x, threadIdx.y, threadIdx.z};\n";
        s += "  const wg_uvec3 wid = {blockIdx.x, blockIdx.y, blockIdx.z};\n";
        s += "  const wg_uvec3 gid = {blockIdx.x * blockDim.x + threadIdx.x, blockIdx.y * blockDim.y + threadIdx.y,"
             " blockIdx.z * blockDim.z + threadIdx.z};\n";
    }
    if (symbolic)
        s += "  const struct { unsigned n0, n1, n2, n3; } params_n = {(unsigned)wg_n0, (unsigned)wg_n1, (unsigned)wg_n2,"
             " (unsigned)wg_n3};\n";
    s += body;
    s += "}\n";
    return s;
}

}  // namespace ah

extern "C" int ah_translate_wgsl(const char *wgsl, char *out, int64_t cap, int64_t *needed) {
    if (!wgsl) return ah::set_error(AH_ERR_INVALID, "ah_translate_wgsl: null source");
    std::string err;
    std::string hip = ah::wgsl_to_hip(wgsl, &err, nullptr);
    if (hip.empty()) return ah::set_error(AH_ERR_COMPILE, "wgsl: %s", err.c_str());
    if (needed) *needed = (int64_t)hip.size() + 1;
    if (out && cap > 0) {
        size_t n = std::min<size_t>((size_t)cap - 1, hip.size());
        memcpy(out, hip.data(), n);
        out[n] = 0;
    }
    return AH_OK;
}
