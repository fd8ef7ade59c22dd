// ckpt.cpp — checkpoint formats for device-resident parameters: safetensors (read/write) and NumPy
// .npy / .npz (read), with the reference's dtype policy.
//
// Reference behaviour followed (paths inside the reference tree):
//   tensor/safetensors/safetensors.go:21-35  load conversions: F32 exact; F64 -> f32 (RTNE); F16 -> f32;
//       BF16 -> f32 by zero-filling the low mantissa; I8/I16/U8/U16 exact; I32/I64/U32/U64 by value with an
//       error past 2^24; BOOL -> 0/1; any other dtype (F8_*, ...) an error naming it;
//   tensor/safetensors/safetensors.go:75-146  save: F32 only, tensor names sorted, header JSON
//       {"name":{"dtype":"F32","shape":[..],"data_offsets":[a,b]},...} padded with spaces to a multiple
//       of 8 bytes, then the data in name order;
//   tensor/safetensors/safetensors.go:37-42   "__metadata__" ignored on load;
//   tensor/npy/npy.go:3-16                   .npy: f32 exact, f64 -> f32, integers by value with the 2^24
//       check, bool -> 0/1, everything else (complex, float16, structured) an error; Fortran order
//       transposed to C order; .npz = ZIP of named .npy entries.
// Everything here is host code: the decoded f32 values are what the trainers upload to their slots.
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <zlib.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "ah_internal.h"

namespace ah {
namespace {

constexpr int64_t kMaxExactInt = int64_t(1) << 24;

struct Entry {
    std::string name;
    std::string dtype;             // safetensors dtype name (npy descr mapped onto the same names)
    std::vector<int64_t> shape;
    int64_t n = 1;
    const unsigned char *data = nullptr;
    int64_t nbytes = 0;
    bool big_endian = false;
    bool fortran = false;
};

int64_t dtype_size(const std::string &t) {
    if (t == "F64" || t == "I64" || t == "U64") return 8;
    if (t == "F32" || t == "I32" || t == "U32") return 4;
    if (t == "F16" || t == "BF16" || t == "I16" || t == "U16") return 2;
    if (t == "I8" || t == "U8" || t == "BOOL") return 1;
    return 0;
}

// ── a small JSON reader for safetensors headers ─────────────────────────────
struct Json {
    const char *p, *e;
    std::string err;
    void ws() { while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++; }
    bool lit(char c) { ws(); if (p < e && *p == c) { p++; return true; } return false; }
    // 4 hex digits at p (advances p); false if malformed
    bool hex4(uint32_t &v) {
        if (e - p < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18)); out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        }
    }
    // A JSON string with every escape JSON defines: \" \\ \/ \b \f \n \r \t and \uXXXX (surrogate
    // pairs joined), decoded to UTF-8. Go's json.Marshal writes <, > and & as \u003c, \u003e, \u0026.
    bool str(std::string &out) {
        ws();
        if (p >= e || *p != '"') { err = "expected a string"; return false; }
        p++;
        out.clear();
        while (p < e && *p != '"') {
            if (*p != '\\') { out += *p++; continue; }
            if (++p >= e) break;
            const char c = *p++;
            switch (c) {
            case '"': case '\\': case '/': out += c; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) { err = "bad \\u escape"; return false; }
                if (cp >= 0xD800 && cp < 0xDC00) {   // high surrogate: a low one must follow
                    uint32_t lo;
                    if (e - p < 6 || p[0] != '\\' || p[1] != 'u') { err = "unpaired surrogate"; return false; }
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) { err = "unpaired surrogate"; return false; }
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    err = "unpaired surrogate";
                    return false;
                }
                utf8(out, cp);
                break;
            }
            default: err = "bad escape"; return false;
            }
        }
        if (p >= e) { err = "unterminated string"; return false; }
        p++;
        return true;
    }
    // An integer bounded by the header's end (the digits are copied out, so strtoll never reads past e).
    bool integer(int64_t &v) {
        ws();
        char buf[32];
        int n = 0;
        while (p + n < e && n < 31 && (p[n] == '-' || (p[n] >= '0' && p[n] <= '9'))) { buf[n] = p[n]; n++; }
        buf[n] = 0;
        char *end = nullptr;
        long long x = strtoll(buf, &end, 10);
        if (n == 0 || end != buf + n || n == 31) { err = "expected an integer"; return false; }
        v = x;
        p += n;
        return true;
    }
    bool int_array(std::vector<int64_t> &v) {
        if (!lit('[')) { err = "expected '['"; return false; }
        v.clear();
        if (lit(']')) return true;
        do {
            int64_t x;
            if (!integer(x)) return false;
            v.push_back(x);
        } while (lit(','));
        if (!lit(']')) { err = "expected ']'"; return false; }
        return true;
    }
    bool skip_value() {   // any JSON value (used for __metadata__)
        ws();
        if (p >= e) return false;
        if (*p == '"') { std::string s; return str(s); }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            p++;
            if (lit(close)) return true;
            do {
                if (open == '{') { std::string k; if (!str(k) || !lit(':')) return false; }
                if (!skip_value()) return false;
            } while (lit(','));
            return lit(close);
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']') p++;
        return true;
    }
};

// ── the reader object ───────────────────────────────────────────────────────
}  // namespace
}  // namespace ah

struct ah_ckpt {
    std::vector<unsigned char> bytes;
    std::vector<ah::Entry> entries;
    std::vector<std::vector<unsigned char>> inflated;   // decompressed .npz members (entries point into them)
};

namespace ah {
namespace {

bool parse_safetensors(ah_ckpt *c, std::string *err) {
    const std::vector<unsigned char> &b = c->bytes;
    if (b.size() < 8) { *err = "file shorter than the 8-byte header length"; return false; }
    uint64_t hl = 0;
    for (int i = 0; i < 8; i++) hl |= (uint64_t)b[i] << (8 * i);
    if (hl > b.size() - 8) { *err = "header length " + std::to_string(hl) + " exceeds the file"; return false; }
    Json j{(const char *)b.data() + 8, (const char *)b.data() + 8 + hl, ""};
    const unsigned char *data = b.data() + 8 + hl;
    const int64_t data_len = (int64_t)(b.size() - 8 - hl);
    if (!j.lit('{')) { *err = "header is not a JSON object"; return false; }
    if (!j.lit('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.lit(':')) { *err = "header: " + j.err; return false; }
            if (name == "__metadata__") {
                if (!j.skip_value()) { *err = "header: bad __metadata__"; return false; }
                continue;
            }
            Entry en;
            en.name = name;
            int64_t off[2] = {-1, -1};
            if (!j.lit('{')) { *err = "header: tensor " + name + " is not an object"; return false; }
            do {
                std::string key;
                if (!j.str(key) || !j.lit(':')) { *err = "header: " + j.err; return false; }
                if (key == "dtype") {
                    if (!j.str(en.dtype)) { *err = "header: " + j.err; return false; }
                } else if (key == "shape") {
                    if (!j.int_array(en.shape)) { *err = "header: " + j.err; return false; }
                } else if (key == "data_offsets") {
                    std::vector<int64_t> o;
                    if (!j.int_array(o) || o.size() != 2) { *err = "header: bad data_offsets for " + name; return false; }
                    off[0] = o[0];
                    off[1] = o[1];
                } else if (!j.skip_value()) {
                    *err = "header: bad value for " + key;
                    return false;
                }
            } while (j.lit(','));
            if (!j.lit('}')) { *err = "header: unterminated tensor " + name; return false; }
            for (int64_t s : en.shape) en.n *= s;
            if (off[0] < 0 || off[1] < off[0] || off[1] > data_len) {
                *err = "tensor " + name + ": data_offsets outside the data section";
                return false;
            }
            en.data = data + off[0];
            en.nbytes = off[1] - off[0];
            c->entries.push_back(en);
        } while (j.lit(','));
        if (!j.lit('}')) { *err = "header: unterminated object"; return false; }
    }
    return true;
}

// One .npy image at b[0..n): fills en (name left to the caller).
bool parse_npy(const unsigned char *b, size_t n, Entry &en, std::string *err) {
    if (n < 10 || memcmp(b, "\x93NUMPY", 6) != 0) { *err = "not an .npy file (bad magic)"; return false; }
    const int major = b[6];
    size_t hl, hs;
    if (major == 1) { hl = b[8] | (b[9] << 8); hs = 10; }
    else if (major == 2 || major == 3) {
        if (n < 12) { *err = "truncated .npy header"; return false; }
        hl = b[8] | (b[9] << 8) | ((size_t)b[10] << 16) | ((size_t)b[11] << 24);
        hs = 12;
    } else { *err = "unsupported .npy version " + std::to_string(major); return false; }
    if (hs + hl > n) { *err = "truncated .npy header"; return false; }
    const std::string h((const char *)b + hs, hl);
    auto field = [&](const char *key) -> std::string {
        size_t k = h.find(std::string("'") + key + "'");
        if (k == std::string::npos) return "";
        size_t colon = h.find(':', k);
        if (colon == std::string::npos) return "";
        size_t v = colon + 1;
        while (v < h.size() && h[v] == ' ') v++;
        if (v < h.size() && h[v] == '\'') {
            size_t end = h.find('\'', v + 1);
            return end == std::string::npos ? "" : h.substr(v + 1, end - v - 1);
        }
        if (v < h.size() && h[v] == '(') {
            size_t end = h.find(')', v);
            return end == std::string::npos ? "" : h.substr(v, end - v + 1);
        }
        size_t end = h.find_first_of(",}", v);
        return h.substr(v, end == std::string::npos ? std::string::npos : end - v);
    };
    const std::string descr = field("descr"), fortran = field("fortran_order"), shape = field("shape");
    if (descr.size() < 3 || shape.empty()) { *err = "malformed .npy header: " + h; return false; }
    const char order = descr[0], kind = descr[1];
    const int size = atoi(descr.c_str() + 2);
    en.big_endian = order == '>';
    en.fortran = fortran.find("True") != std::string::npos;
    std::string t;
    if (kind == 'f' && size == 4) t = "F32";
    else if (kind == 'f' && size == 8) t = "F64";
    else if (kind == 'i' && (size == 1 || size == 2 || size == 4 || size == 8)) t = "I" + std::to_string(8 * size);
    else if (kind == 'u' && (size == 1 || size == 2 || size == 4 || size == 8)) t = "U" + std::to_string(8 * size);
    else if (kind == 'b' && size == 1) t = "BOOL";
    else if (kind == 'c') { *err = "unsupported numpy dtype " + descr + " (complex)"; return false; }
    else { *err = "unsupported numpy dtype " + descr; return false; }
    en.dtype = t;
    en.shape.clear();
    for (size_t i = 1; i < shape.size();) {   // "(3, 4)", "(4,)", "()"
        while (i < shape.size() && (shape[i] == ' ' || shape[i] == ',')) i++;
        if (i >= shape.size() || shape[i] == ')') break;
        char *end = nullptr;
        long long v = strtoll(shape.c_str() + i, &end, 10);
        if (end == shape.c_str() + i) { *err = "malformed .npy shape " + shape; return false; }
        en.shape.push_back(v);
        i = end - shape.c_str();
    }
    en.n = 1;
    for (int64_t s : en.shape) en.n *= s;
    en.data = b + hs + hl;
    en.nbytes = (int64_t)(n - hs - hl);
    if (en.nbytes < en.n * dtype_size(t)) { *err = "truncated .npy data"; return false; }
    en.nbytes = en.n * dtype_size(t);
    return true;
}

uint32_t rd32(const unsigned char *p) { return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24); }
uint16_t rd16(const unsigned char *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

bool parse_npz(ah_ckpt *c, std::string *err) {
    const std::vector<unsigned char> &b = c->bytes;
    if (b.size() < 22) { *err = "not a ZIP archive"; return false; }
    size_t eocd = std::string::npos;
    for (size_t i = b.size() - 22; i + 1 > 0; i--) {
        if (rd32(&b[i]) == 0x06054b50u) { eocd = i; break; }
        if (i == 0 || b.size() - i > 22 + 65535) break;
    }
    if (eocd == std::string::npos) { *err = "ZIP end of central directory not found"; return false; }
    const uint16_t count = rd16(&b[eocd + 10]);
    size_t cd = rd32(&b[eocd + 16]);
    for (int k = 0; k < count; k++) {
        if (cd + 46 > b.size() || rd32(&b[cd]) != 0x02014b50u) { *err = "bad ZIP central directory"; return false; }
        const uint16_t method = rd16(&b[cd + 10]);
        const uint32_t csize = rd32(&b[cd + 20]), usize = rd32(&b[cd + 24]);
        const uint16_t nlen = rd16(&b[cd + 28]), xlen = rd16(&b[cd + 30]), clen = rd16(&b[cd + 32]);
        const uint32_t lho = rd32(&b[cd + 42]);
        if (cd + 46 + (size_t)nlen + xlen + clen > b.size()) { *err = "bad ZIP central directory entry"; return false; }
        std::string name((const char *)&b[cd + 46], nlen);
        cd += 46 + nlen + xlen + clen;
        if (method != 0 && method != 8) {
            *err = "npz entry " + name + ": ZIP method " + std::to_string(method) + " (stored and deflate are read)";
            return false;
        }
        if (csize == 0xFFFFFFFFu || usize == 0xFFFFFFFFu || lho == 0xFFFFFFFFu) {
            *err = "npz entry " + name + " needs ZIP64, which is not read";
            return false;
        }
        if ((size_t)lho + 30 > b.size() || rd32(&b[lho]) != 0x04034b50u) { *err = "bad ZIP local header for " + name; return false; }
        const size_t start = (size_t)lho + 30 + rd16(&b[lho + 26]) + rd16(&b[lho + 28]);
        if (start + csize > b.size()) { *err = "truncated npz entry " + name; return false; }
        const unsigned char *member = &b[start];
        size_t member_size = csize;
        if (method == 8) {   // raw deflate, as np.savez_compressed writes
            std::vector<unsigned char> out(std::max<uint32_t>(usize, 1));
            z_stream zs;
            memset(&zs, 0, sizeof zs);
            if (inflateInit2(&zs, -MAX_WBITS) != Z_OK) { *err = "inflate init failed"; return false; }
            zs.next_in = const_cast<unsigned char *>(member);
            zs.avail_in = csize;
            zs.next_out = out.data();
            zs.avail_out = usize;
            const int zr = inflate(&zs, Z_FINISH);
            const size_t got = zs.total_out;
            inflateEnd(&zs);
            if (zr != Z_STREAM_END || got != usize) { *err = "npz entry " + name + ": corrupt deflate data"; return false; }
            c->inflated.push_back(std::move(out));
            member = c->inflated.back().data();
            member_size = usize;
        }
        Entry en;
        if (!parse_npy(member, member_size, en, err)) { *err = name + ": " + *err; return false; }
        if (name.size() > 4 && name.compare(name.size() - 4, 4, ".npy") == 0) name.resize(name.size() - 4);
        en.name = name;
        c->entries.push_back(en);
    }
    return true;
}

template <class T>
T load_le(const unsigned char *p, bool big) {
    T v;
    if (!big) { memcpy(&v, p, sizeof(T)); return v; }
    unsigned char r[sizeof(T)];
    for (size_t i = 0; i < sizeof(T); i++) r[i] = p[sizeof(T) - 1 - i];
    memcpy(&v, r, sizeof(T));
    return v;
}

// Element i (C order) of en as f32, following the dtype policy; false + message on an error.
bool decode_all(const Entry &en, float *out, std::string *err) {
    const int64_t es = dtype_size(en.dtype);
    if (es == 0) { *err = "unsupported dtype " + en.dtype + " for tensor " + en.name; return false; }
    if (en.nbytes != en.n * es) {
        *err = "tensor " + en.name + ": " + std::to_string(en.nbytes) + " data bytes for " + std::to_string(en.n) +
               " elements of " + en.dtype;
        return false;
    }
    // Fortran order: the stored element at flat position f has C index with reversed strides.
    const int rank = (int)en.shape.size();
    auto src_index = [&](int64_t ci) -> int64_t {
        if (!en.fortran || rank < 2) return ci;
        int64_t rem = ci, fi = 0, fstride = 1;
        std::vector<int64_t> idx(rank);
        for (int d = rank - 1; d >= 0; d--) { idx[d] = rem % en.shape[d]; rem /= en.shape[d]; }
        for (int d = 0; d < rank; d++) { fi += idx[d] * fstride; fstride *= en.shape[d]; }
        return fi;
    };
    const bool be = en.big_endian;
    for (int64_t i = 0; i < en.n; i++) {
        const unsigned char *p = en.data + src_index(i) * es;
        const std::string &t = en.dtype;
        double v = 0;
        int64_t iv = 0;
        bool is_int = false;
        if (t == "F32") { out[i] = load_le<float>(p, be); continue; }
        if (t == "F64") { out[i] = (float)load_le<double>(p, be); continue; }
        if (t == "F16") { out[i] = ah_f16_to_f32(load_le<uint16_t>(p, be)); continue; }
        if (t == "BF16") {
            const uint32_t bits = (uint32_t)load_le<uint16_t>(p, be) << 16;
            memcpy(&out[i], &bits, 4);
            continue;
        }
        if (t == "BOOL") { out[i] = p[0] ? 1.0f : 0.0f; continue; }
        if (t == "I8") { iv = (int8_t)p[0]; is_int = true; }
        else if (t == "U8") { iv = p[0]; is_int = true; }
        else if (t == "I16") { iv = load_le<int16_t>(p, be); is_int = true; }
        else if (t == "U16") { iv = load_le<uint16_t>(p, be); is_int = true; }
        else if (t == "I32") { iv = load_le<int32_t>(p, be); is_int = true; }
        else if (t == "U32") { iv = load_le<uint32_t>(p, be); is_int = true; }
        else if (t == "I64") { iv = load_le<int64_t>(p, be); is_int = true; }
        else if (t == "U64") {
            const uint64_t u = load_le<uint64_t>(p, be);
            if (u > (uint64_t)kMaxExactInt) {
                *err = "tensor " + en.name + ": value " + std::to_string(u) + " exceeds the exact float32 integer range (2^24)";
                return false;
            }
            iv = (int64_t)u;
            is_int = true;
        }
        if (is_int) {
            if (iv > kMaxExactInt || iv < -kMaxExactInt) {
                *err = "tensor " + en.name + ": value " + std::to_string(iv) + " exceeds the exact float32 integer range (2^24)";
                return false;
            }
            out[i] = (float)iv;
            continue;
        }
        (void)v;
    }
    return true;
}

void json_escape(std::string &o, const std::string &s) {
    for (char ch : s) {
        if (ch == '"' || ch == '\\') { o += '\\'; o += ch; }
        else if ((unsigned char)ch < 0x20) { char buf[8]; snprintf(buf, sizeof buf, "\\u%04x", ch); o += buf; }
        else o += ch;
    }
}

}  // namespace
}  // namespace ah

using namespace ah;

extern "C" {

int ah_ckpt_open(const char *path, ah_ckpt **out) {
    if (!path || !out) return set_error(AH_ERR_INVALID, "ah_ckpt_open: null argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return set_error(AH_ERR_INVALID, "checkpoint: cannot open %s", path);
    auto *c = new ah_ckpt();
    unsigned char buf[1 << 16];
    size_t r;
    while ((r = fread(buf, 1, sizeof buf, f)) > 0) c->bytes.insert(c->bytes.end(), buf, buf + r);
    fclose(f);
    std::string err;
    bool ok;
    const std::string p(path);
    if (c->bytes.size() >= 6 && memcmp(c->bytes.data(), "\x93NUMPY", 6) == 0) {
        Entry en;
        ok = parse_npy(c->bytes.data(), c->bytes.size(), en, &err);
        if (ok) {
            size_t slash = p.find_last_of('/');
            std::string base = p.substr(slash == std::string::npos ? 0 : slash + 1);
            if (base.size() > 4 && base.compare(base.size() - 4, 4, ".npy") == 0) base.resize(base.size() - 4);
            en.name = base;
            c->entries.push_back(en);
        }
    } else if (c->bytes.size() >= 4 && rd32(c->bytes.data()) == 0x04034b50u) {
        ok = parse_npz(c, &err);
    } else {
        ok = parse_safetensors(c, &err);
    }
    if (!ok) {
        delete c;
        return set_error(AH_ERR_INVALID, "checkpoint %s: %s", path, err.c_str());
    }
    *out = c;
    return AH_OK;
}

int32_t ah_ckpt_count(const ah_ckpt *c) { return c ? (int32_t)c->entries.size() : 0; }

int ah_ckpt_entry(const ah_ckpt *c, int32_t i, const char **name, const char **dtype, int32_t *rank,
                  const int64_t **shape, int64_t *n_elems) {
    if (!c || i < 0 || i >= (int32_t)c->entries.size()) return set_error(AH_ERR_INVALID, "ah_ckpt_entry: bad index");
    const Entry &e = c->entries[i];
    if (name) *name = e.name.c_str();
    if (dtype) *dtype = e.dtype.c_str();
    if (rank) *rank = (int32_t)e.shape.size();
    if (shape) *shape = e.shape.data();
    if (n_elems) *n_elems = e.n;
    return AH_OK;
}

int ah_ckpt_read(const ah_ckpt *c, int32_t i, float *out, int64_t n) {
    if (!c || !out || i < 0 || i >= (int32_t)c->entries.size()) return set_error(AH_ERR_INVALID, "ah_ckpt_read: bad argument");
    const Entry &e = c->entries[i];
    if (n != e.n) return set_error(AH_ERR_INVALID, "ah_ckpt_read: tensor %s has %lld elements, buffer %lld", e.name.c_str(),
                                   (long long)e.n, (long long)n);
    std::string err;
    if (!decode_all(e, out, &err)) return set_error(AH_ERR_INVALID, "checkpoint: %s", err.c_str());
    return AH_OK;
}

void ah_ckpt_close(ah_ckpt *c) { delete c; }

int ah_safetensors_save(const char *path, int32_t n, const char *const *names, const float *const *data,
                        const int64_t *const *shapes, const int32_t *ranks) {
    if (!path || n < 0 || (n > 0 && (!names || !data || !shapes || !ranks)))
        return set_error(AH_ERR_INVALID, "ah_safetensors_save: null argument");
    std::vector<int> order(n);
    for (int i = 0; i < n; i++) order[i] = i;
    std::sort(order.begin(), order.end(), [&](int a, int b) { return strcmp(names[a], names[b]) < 0; });
    for (int i = 1; i < n; i++)
        if (strcmp(names[order[i - 1]], names[order[i]]) == 0) return set_error(AH_ERR_INVALID, "safetensors: duplicate name %s", names[order[i]]);
    std::string h = "{";
    int64_t off = 0;
    std::vector<int64_t> counts(n);
    for (int k = 0; k < n; k++) {
        const int i = order[k];
        int64_t cnt = 1;
        for (int d = 0; d < ranks[i]; d++) cnt *= shapes[i][d];
        counts[i] = cnt;
        if (k) h += ",";
        h += "\"";
        json_escape(h, names[i]);
        h += "\":{\"dtype\":\"F32\",\"shape\":[";
        for (int d = 0; d < ranks[i]; d++) h += (d ? "," : "") + std::to_string(shapes[i][d]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + 4 * cnt) + "]}";
        off += 4 * cnt;
    }
    h += "}";
    while (h.size() % 8) h += ' ';
    FILE *f = fopen(path, "wb");
    if (!f) return set_error(AH_ERR_INVALID, "safetensors: cannot create %s", path);
    unsigned char len[8];
    for (int i = 0; i < 8; i++) len[i] = (unsigned char)((uint64_t)h.size() >> (8 * i));
    bool ok = fwrite(len, 1, 8, f) == 8 && fwrite(h.data(), 1, h.size(), f) == h.size();
    for (int k = 0; k < n && ok; k++) {
        const int i = order[k];
        ok = fwrite(data[i], 4, (size_t)counts[i], f) == (size_t)counts[i];   // little-endian host
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) return set_error(AH_ERR_INVALID, "safetensors: write to %s failed", path);
    return AH_OK;
}

}  // extern "C"
