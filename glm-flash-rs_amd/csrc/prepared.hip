// Prepared-weight loader: the reference's on-disk weight format (glm-flash-rs src/prepared.rs) read into device
// memory, so that the expert engines can run on real EXL3 checkpoints converted by the reference's tooling.
//
// Format (prepared.rs:15-40, 101-132, 186-230): a JSON manifest {format: 1, file_size, chunk, chunk_sha256[],
// storages[{offset, nbytes, dev}], tree, key} next to `data.bin`. Storages are byte ranges of data.bin, ascending and
// non-overlapping. The tree is a typed object graph: {"T": storage, dtype, shape, stride, off, dev} is a tensor view
// (element offset and strides into its storage), {"O": type, "f": {fields}} an object, {"L"|"U": [...]} a sequence,
// {"D": [[key, value], ...]} a dict, {"P": ...} / {"dev": ...} a primitive. Tensor paths are built as the reference
// builds them ("weights.layers[3].moe.experts.gt"). Loading reads data.bin in `chunk`-byte pieces through pinned
// staging, checks each needed piece's SHA-256 against the manifest, and copies the overlapping storage bytes.
//
// Not carried over: the reference's model-identity checks (model name, TP4 rank, GLM geometry; prepared.rs:151-185)
// belong to its full model, not to the expert path; callers that need them read the manifest's `key` themselves.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>
#include <fcntl.h>
#include <unistd.h>
#ifndef __HIP_DEVICE_COMPILE__
#include <cpuid.h>
#include <immintrin.h>
#endif

#include <algorithm>
#include <chrono>
#include <deque>
#include <future>
#include <thread>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/gfr_moe.h"

namespace gfr {
int set_error(int code, const std::string& msg);   // gfr_moe_api.hip (the thread's gfr_last_error)
}

namespace {

// ---- SHA-256 (FIPS 180-4) ---------------------------------------------------------------------------------------
static const uint32_t SHA256_K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

#ifndef __HIP_DEVICE_COMPILE__
// The same compression with the x86 SHA extensions (host only): the state as (A, B, E, F) and (C, D, G, H), two
// rounds a sha256rnds2, the message schedule four words at a time (sha256msg1 / sha256msg2), after Intel's published
// description of the instructions. Used when CPUID reports them; about 4-5x the scalar rate a thread.
static bool cpu_has_sha() {
    unsigned a, b, c, d;
    return __get_cpuid_count(7, 0, &a, &b, &c, &d) && ((b >> 29) & 1);
}
__attribute__((target("sha,sse4.1,ssse3"))) static void sha256_blocks_ni(uint32_t h[8], const uint8_t* p,
                                                                          size_t nblocks) {
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bull, 0x0405060700010203ull);
    __m128i t = _mm_loadu_si128(reinterpret_cast<const __m128i*>(h));        // (A, B, C, D)
    __m128i s1 = _mm_loadu_si128(reinterpret_cast<const __m128i*>(h + 4));   // (E, F, G, H)
    t = _mm_shuffle_epi32(t, 0xB1);                                           // (B, A, D, C)
    s1 = _mm_shuffle_epi32(s1, 0x1B);                                         // (H, G, F, E)
    __m128i s0 = _mm_alignr_epi8(t, s1, 8);                                   // (F, E, B, A): ABEF
    s1 = _mm_blend_epi16(s1, t, 0xF0);                                        // (H, G, D, C): CDGH
    for (; nblocks; --nblocks, p += 64) {
        const __m128i s0_in = s0, s1_in = s1;
        __m128i w[4];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __m128i wi;
            if (i < 4) {
                wi = _mm_shuffle_epi8(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p + 16 * i)), bswap);
            } else {   // W[t] from W[t-16..t-13] (msg1), W[t-7..t-4] and W[t-2..t-1] (msg2)
                __m128i x = _mm_sha256msg1_epu32(w[(i - 4) & 3], w[(i - 3) & 3]);
                x = _mm_add_epi32(x, _mm_alignr_epi8(w[(i - 1) & 3], w[(i - 2) & 3], 4));
                wi = _mm_sha256msg2_epu32(x, w[(i - 1) & 3]);
            }
            w[i & 3] = wi;
            __m128i m = _mm_add_epi32(wi, _mm_loadu_si128(reinterpret_cast<const __m128i*>(SHA256_K + 4 * i)));
            s1 = _mm_sha256rnds2_epu32(s1, s0, m);
            m = _mm_shuffle_epi32(m, 0x0E);
            s0 = _mm_sha256rnds2_epu32(s0, s1, m);
        }
        s0 = _mm_add_epi32(s0, s0_in);
        s1 = _mm_add_epi32(s1, s1_in);
    }
    t = _mm_shuffle_epi32(s0, 0x1B);                                          // (A, B, E, F) -> FEBA order
    s1 = _mm_shuffle_epi32(s1, 0xB1);
    s0 = _mm_blend_epi16(t, s1, 0xF0);                                        // (A, B, C, D)
    s1 = _mm_alignr_epi8(s1, t, 8);                                           // (E, F, G, H)
    _mm_storeu_si128(reinterpret_cast<__m128i*>(h), s0);
    _mm_storeu_si128(reinterpret_cast<__m128i*>(h + 4), s1);
}
#endif

struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t buf[64];
    uint64_t total = 0;
    size_t fill = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t* p) {
        const uint32_t* k = SHA256_K;
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    // whole blocks: the SHA extensions when the CPU has them (GFR_SHA_SCALAR=1 forces the scalar rounds)
    void blocks(const uint8_t* p, size_t n) {
#ifndef __HIP_DEVICE_COMPILE__
        static const bool ni = cpu_has_sha() && !getenv("GFR_SHA_SCALAR");
        if (ni) { sha256_blocks_ni(h, p, n); return; }
#endif
        for (; n; --n, p += 64) block(p);
    }
    void update(const void* data, size_t len) {
        const uint8_t* p = static_cast<const uint8_t*>(data);
        total += len;
        if (fill) {
            const size_t n = std::min(len, 64 - fill);
            memcpy(buf + fill, p, n);
            fill += n; p += n; len -= n;
            if (fill == 64) { blocks(buf, 1); fill = 0; }
        }
        if (len >= 64) { blocks(p, len / 64); p += len / 64 * 64; len %= 64; }
        if (len) { memcpy(buf, p, len); fill = len; }
    }
    std::string hex() {
        const uint64_t bits = total * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t lenb[8];
        for (int i = 0; i < 8; ++i) lenb[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(lenb, 8);
        char out[65];
        for (int i = 0; i < 8; ++i) snprintf(out + 8 * i, 9, "%08x", h[i]);
        return std::string(out, 64);
    }
};

// ---- a small JSON reader (objects keep their key order; integers keep all 64 bits) --------------------------------
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    bool is_uint = false;   // a non-negative integer literal that fits in 64 bits
    uint64_t u = 0;
    std::string s;          // Str: the string; Num: the literal text
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;

    const Json* get(const char* key) const {
        if (kind != Obj) return nullptr;
        for (auto& kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    // serde_json's compact Display of a value, for dict keys in paths (prepared.rs:122)
    std::string display() const {
        switch (kind) {
            case Null: return "null";
            case Bool: return b ? "true" : "false";
            case Num: return s;
            case Str: {
                std::string r = "\"";
                for (char c : s) {
                    if (c == '"' || c == '\\') { r += '\\'; r += c; }
                    else if (c == '\n') r += "\\n";
                    else if (c == '\t') r += "\\t";
                    else if (c == '\r') r += "\\r";
                    else if ((unsigned char)c < 0x20) { char t[8]; snprintf(t, sizeof t, "\\u%04x", c); r += t; }
                    else r += c;
                }
                return r + "\"";
            }
            case Arr: {
                std::string r = "[";
                for (size_t i = 0; i < a.size(); ++i) r += (i ? "," : "") + a[i].display();
                return r + "]";
            }
            case Obj: {
                std::string r = "{";
                for (size_t i = 0; i < o.size(); ++i) r += (i ? "," : "") + Json{Str, false, false, 0, o[i].first}.display() + ":" + o[i].second.display();
                return r + "}";
            }
        }
        return "";
    }
};

struct Parser {
    const char* p;
    const char* end;
    std::string err;
    int depth = 0;

    void ws() { while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p; }
    bool fail(const char* m) { if (err.empty()) err = m; return false; }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n)) return fail("bad literal");
        p += n;
        return true;
    }
    bool str(std::string& out) {
        if (p >= end || *p != '"') return fail("expected string");
        ++p;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') { out += c; continue; }
            if (p >= end) return fail("bad escape");
            c = *p++;
            switch (c) {
                case '"': case '\\': case '/': out += c; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (end - p < 4) return fail("bad \\u escape");
                    unsigned cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p++;
                        cp = cp * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                        : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
                        if (cp > 0xffff) return fail("bad \\u escape");
                    }
                    if (cp < 0x80) out += (char)cp;
                    else if (cp < 0x800) { out += (char)(0xc0 | cp >> 6); out += (char)(0x80 | (cp & 0x3f)); }
                    else { out += (char)(0xe0 | cp >> 12); out += (char)(0x80 | ((cp >> 6) & 0x3f)); out += (char)(0x80 | (cp & 0x3f)); }
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 256) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        bool ok = true;
        const char c = *p;
        if (c == '{') {
            v.kind = Json::Obj;
            ++p; ws();
            if (p < end && *p == '}') { ++p; }
            else for (;;) {
                std::string k;
                ws();
                if (!str(k)) { ok = false; break; }
                ws();
                if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
                ++p;
                v.o.emplace_back(std::move(k), Json{});
                if (!value(v.o.back().second)) { ok = false; break; }
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == '}') { ++p; break; }
                ok = fail("expected ',' or '}'");
                break;
            }
        } else if (c == '[') {
            v.kind = Json::Arr;
            ++p; ws();
            if (p < end && *p == ']') { ++p; }
            else for (;;) {
                v.a.emplace_back();
                if (!value(v.a.back())) { ok = false; break; }
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') { ++p; break; }
                ok = fail("expected ',' or ']'");
                break;
            }
        } else if (c == '"') {
            v.kind = Json::Str;
            ok = str(v.s);
        } else if (c == 't') { v.kind = Json::Bool; v.b = true; ok = lit("true"); }
        else if (c == 'f') { v.kind = Json::Bool; v.b = false; ok = lit("false"); }
        else if (c == 'n') { v.kind = Json::Null; ok = lit("null"); }
        else if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Json::Num;
            const char* q = p;
            while (p < end && (strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) ++p;
            v.s.assign(q, p);
            bool digits = !v.s.empty();
            for (char d : v.s) digits = digits && d >= '0' && d <= '9';
            if (digits) {
                uint64_t x = 0;
                bool over = false;
                for (char d : v.s) over |= __builtin_mul_overflow(x, 10u, &x) || __builtin_add_overflow(x, (uint64_t)(d - '0'), &x);
                v.is_uint = !over;
                v.u = x;
            }
        } else ok = fail("unexpected character");
        --depth;
        return ok;
    }
};

bool parse_json(const std::string& text, Json& out, std::string& err) {
    Parser ps{text.data(), text.data() + text.size(), {}};
    if (!ps.value(out)) { err = ps.err; return false; }
    ps.ws();
    if (ps.p != ps.end) { err = "trailing characters"; return false; }
    return true;
}

// ---- the prepared model ---------------------------------------------------------------------------------------
struct Storage { uint64_t offset, nbytes; bool cuda; };
struct Tensor {
    uint64_t storage;
    std::string dtype;
    std::vector<uint64_t> shape, stride;
    uint64_t off;
    bool cuda;
};

int err(const std::string& m) { return gfr::set_error(GFR_EINVAL, m); }

// Tensor::element_bytes (prepared.rs:42-50)
int element_bytes(const std::string& dtype, uint64_t& eb) {
    if (dtype == "bool" || dtype == "uint8" || dtype == "int8" || dtype == "float8_e4m3fn" || dtype == "float8_e5m2") eb = 1;
    else if (dtype == "bfloat16" || dtype == "float16" || dtype == "int16" || dtype == "uint16") eb = 2;
    else if (dtype == "float32" || dtype == "int32" || dtype == "uint32") eb = 4;
    else if (dtype == "float64" || dtype == "int64" || dtype == "uint64") eb = 8;
    else return err("unsupported dtype " + dtype);
    return 0;
}

// Tensor::extent (prepared.rs:51-71): bytes from the storage start to the view's last element, checked
int extent(const Tensor& t, uint64_t& bytes) {
    uint64_t eb;
    if (int rc = element_bytes(t.dtype, eb)) return rc;
    if (t.shape.size() != t.stride.size()) return err("shape/stride rank differs");
    if (std::find(t.shape.begin(), t.shape.end(), 0) != t.shape.end()) {
        if (__builtin_mul_overflow(t.off, eb, &bytes)) return err("empty tensor overflow");
        return 0;
    }
    uint64_t last = t.off;
    for (size_t i = 0; i < t.shape.size(); ++i) {
        uint64_t step;
        if (__builtin_mul_overflow(t.shape[i] - 1, t.stride[i], &step)) return err("tensor stride overflow");
        if (__builtin_add_overflow(last, step, &last)) return err("tensor extent overflow");
    }
    if (__builtin_add_overflow(last, (uint64_t)1, &last) || __builtin_mul_overflow(last, eb, &bytes))
        return err("tensor bytes overflow");
    return 0;
}

bool get_u64(const Json* j, uint64_t& v) {
    if (!j || j->kind != Json::Num || !j->is_uint) return false;
    v = j->u;
    return true;
}

// walk (prepared.rs:101-132)
int walk(const Json& node, const std::string& path, std::map<std::string, Tensor>& tensors) {
    if (node.kind != Json::Obj) return err("prepared node is not an object: " + path);
    if (node.get("T")) {
        Tensor t;
        const Json* dt = node.get("dtype");
        const Json* sh = node.get("shape");
        const Json* st = node.get("stride");
        const Json* dev = node.get("dev");
        if (!get_u64(node.get("T"), t.storage) || !dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr ||
            !st || st->kind != Json::Arr || !get_u64(node.get("off"), t.off) || !dev || dev->kind != Json::Str)
            return err("bad tensor node " + path);
        t.dtype = dt->s;
        for (auto& x : sh->a) { uint64_t v; if (!get_u64(&x, v)) return err("bad shape " + path); t.shape.push_back(v); }
        for (auto& x : st->a) { uint64_t v; if (!get_u64(&x, v)) return err("bad stride " + path); t.stride.push_back(v); }
        if (dev->s != "cuda" && dev->s != "cpu") return err("unknown tensor device " + path);
        t.cuda = dev->s == "cuda";
        tensors[path] = t;
    } else if (const Json* f = node.get("f")) {
        const Json* o = node.get("O");
        if (!o || o->kind != Json::Str) return err("untyped object " + path);
        if (f->kind != Json::Obj) return err("object fields " + path);
        for (auto& kv : f->o)
            if (int rc = walk(kv.second, path + "." + kv.first, tensors)) return rc;
    } else if (const Json* l = node.get("L") ? node.get("L") : node.get("U")) {
        if (l->kind != Json::Arr) return err("sequence " + path);
        for (size_t i = 0; i < l->a.size(); ++i)
            if (int rc = walk(l->a[i], path + "[" + std::to_string(i) + "]", tensors)) return rc;
    } else if (const Json* d = node.get("D")) {
        if (d->kind != Json::Arr) return err("dict " + path);
        for (auto& pr : d->a) {
            if (pr.kind != Json::Arr) return err("dict pair " + path);
            if (pr.a.size() != 2) return err("dict pair length " + path);
            if (int rc = walk(pr.a[1], path + "[" + pr.a[0].display() + "]", tensors)) return rc;
        }
    } else if (node.get("N")) {
        return err("NumPy storage is unsupported: " + path);
    } else if (!(node.o.size() == 1 && (node.get("P") || node.get("dev")))) {
        return err("unknown prepared node " + path);
    }
    return 0;
}

}  // namespace

struct gfr_prepared {
    std::string data_path;
    uint64_t file_size = 0, chunk = 0;
    std::vector<std::string> chunk_sha256;
    std::vector<Storage> storages;
    std::map<std::string, Tensor> tensors;
    std::vector<std::string> names;              // tensors in path order
    std::vector<void*> dev;                      // loaded cuda storages (null: absent)
    std::vector<std::vector<uint8_t>> host;      // loaded cpu storages
    std::vector<bool> loaded;
    uint64_t loaded_bytes = 0;
    double load_seconds = 0;
};

namespace {

void release(gfr_prepared* p) {
    for (void*& d : p->dev)
        if (d) { (void)hipFree(d); d = nullptr; }
    p->host.assign(p->storages.size(), {});
    p->loaded.assign(p->storages.size(), false);
}

const Tensor* find(const gfr_prepared* p, const char* path) {
    if (!p || !path) return nullptr;
    auto it = p->tensors.find(path);
    return it == p->tensors.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

int gfr_sha256_hex(const void* data, uint64_t len, char* out65) {
    if ((!data && len) || !out65) return err("null argument");
    Sha256 h;
    h.update(data, len);
    const std::string x = h.hex();
    memcpy(out65, x.c_str(), 65);
    return 0;
}

int gfr_tensor_extent(const char* dtype, const uint64_t* shape, const uint64_t* stride, int shape_rank,
                      int stride_rank, uint64_t off, uint64_t* bytes) {
    if (!dtype || !bytes || shape_rank < 0 || stride_rank < 0 || (shape_rank && !shape) || (stride_rank && !stride))
        return err("bad tensor description");
    Tensor t{0, dtype, std::vector<uint64_t>(shape, shape + shape_rank), std::vector<uint64_t>(stride, stride + stride_rank),
             off, true};
    return extent(t, *bytes);
}

// Prepared::open_parts (prepared.rs:186-230) with the tree walk of Prepared::open (:171-172)
int gfr_prepared_open(gfr_prepared** out, const char* manifest_path) {
    if (!out || !manifest_path) return err("null argument");
    *out = nullptr;
    FILE* f = fopen(manifest_path, "rb");
    if (!f) return err(std::string("cannot open manifest ") + manifest_path);
    std::string text;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    fclose(f);
    Json m;
    std::string perr;
    if (!parse_json(text, m, perr)) return err("manifest is not JSON: " + perr);
    if (m.kind != Json::Obj) return err("manifest is not an object");
    uint64_t format;
    if (!get_u64(m.get("format"), format) || format != 1) return err("unsupported prepared format");
    std::unique_ptr<gfr_prepared> p(new gfr_prepared);
    if (!get_u64(m.get("file_size"), p->file_size) || !get_u64(m.get("chunk"), p->chunk)) return err("bad manifest sizes");
    if (p->chunk == 0 || p->chunk > 128ull * 1024 * 1024) return err("invalid chunk size");
    const Json* hs = m.get("chunk_sha256");
    if (!hs || hs->kind != Json::Arr) return err("missing chunk_sha256");
    for (auto& h : hs->a) {
        if (h.kind != Json::Str) return err("bad chunk hash");
        p->chunk_sha256.push_back(h.s);
    }
    if ((uint64_t)p->chunk_sha256.size() != (p->file_size + p->chunk - 1) / p->chunk) return err("chunk hash count");
    const std::string mp(manifest_path);
    const size_t slash = mp.find_last_of('/');
    p->data_path = (slash == std::string::npos ? std::string() : mp.substr(0, slash + 1)) + "data.bin";
    FILE* d = fopen(p->data_path.c_str(), "rb");
    if (!d) return err("cannot open " + p->data_path);
    fseeko(d, 0, SEEK_END);
    const uint64_t dsize = (uint64_t)ftello(d);
    fclose(d);
    if (dsize != p->file_size) return err("data file size mismatch");
    const Json* ss = m.get("storages");
    if (!ss || ss->kind != Json::Arr) return err("missing storages");
    uint64_t prev = 0;
    for (auto& s : ss->a) {
        Storage st;
        const Json* dev = s.get("dev");
        if (!get_u64(s.get("offset"), st.offset) || !get_u64(s.get("nbytes"), st.nbytes) || !dev || dev->kind != Json::Str)
            return err("bad storage entry");
        if (st.nbytes == 0 || st.offset < prev) return err("empty/overlapping/out-of-order storage");
        if (__builtin_add_overflow(st.offset, st.nbytes, &prev)) return err("storage overflow");
        if (prev > p->file_size) return err("storage outside data file");
        if (dev->s != "cuda" && dev->s != "cpu") return err("unknown storage device");
        st.cuda = dev->s == "cuda";
        p->storages.push_back(st);
    }
    const Json* tree = m.get("tree");
    if (!tree) return err("missing tree");
    if (int rc = walk(*tree, "weights", p->tensors)) return rc;
    for (auto& kv : p->tensors) {
        const Tensor& t = kv.second;
        if (t.storage >= p->storages.size()) return err("missing storage for " + kv.first);
        const Storage& s = p->storages[t.storage];
        uint64_t ext;
        if (int rc = extent(t, ext)) return rc;
        if (ext > s.nbytes) return err("tensor " + kv.first + " escapes storage");
        if (t.cuda != s.cuda) return err("tensor " + kv.first + " changes device");
        p->names.push_back(kv.first);
    }
    if (p->tensors.empty()) return err("no tensors");
    p->dev.assign(p->storages.size(), nullptr);
    release(p.get());
    *out = p.release();
    return 0;
}

int gfr_prepared_tensor_count(const gfr_prepared* p) { return p ? (int)p->names.size() : 0; }

const char* gfr_prepared_tensor_name(const gfr_prepared* p, int i) {
    return p && i >= 0 && i < (int)p->names.size() ? p->names[i].c_str() : nullptr;
}

// Prepared::tensor (prepared.rs:231-235) and Tensor::extent
int gfr_prepared_tensor(const gfr_prepared* p, const char* path, gfr_tensor_info* info) {
    const Tensor* t = find(p, path);
    if (!t) return err(std::string("missing tensor ") + (path ? path : "(null)"));
    if (!info) return err("null info");
    memset(info, 0, sizeof *info);
    if (t->shape.size() > GFR_TENSOR_MAX_RANK) return err(std::string("rank too large for ") + path);
    info->storage = (int)t->storage;
    snprintf(info->dtype, sizeof info->dtype, "%s", t->dtype.c_str());
    info->rank = (int)t->shape.size();
    for (size_t i = 0; i < t->shape.size(); ++i) { info->shape[i] = t->shape[i]; info->stride[i] = t->stride[i]; }
    info->off = t->off;
    info->cuda = t->cuda ? 1 : 0;
    return extent(*t, info->extent_bytes);
}

// Prepared::expect (prepared.rs:236-248): dtype, shape, device cuda, contiguous row-major
int gfr_prepared_expect(const gfr_prepared* p, const char* path, const char* dtype, const uint64_t* shape, int rank) {
    const Tensor* t = find(p, path);
    if (!t) return err(std::string("missing tensor ") + (path ? path : "(null)"));
    if (!dtype || rank < 0 || (rank && !shape) || t->dtype != dtype || (int)t->shape.size() != rank ||
        !std::equal(t->shape.begin(), t->shape.end(), shape) || !t->cuda)
        return err(std::string("unsupported tensor ") + path);
    uint64_t stride = 1;
    for (int i = rank - 1; i >= 0; --i) {
        if (t->stride[i] != stride) return err(std::string("noncontiguous tensor ") + path);
        stride *= t->shape[i];
    }
    return 0;
}

// Prepared::read_tensor_segment (prepared.rs:253-266): bytes [offset, offset + len) of the view's extent, from disk
int gfr_prepared_read_tensor(const gfr_prepared* p, const char* path, uint64_t offset, uint64_t len, void* out) {
    const Tensor* t = find(p, path);
    if (!t) return err(std::string("missing tensor ") + (path ? path : "(null)"));
    uint64_t ext, eb;
    if (int rc = extent(*t, ext)) return rc;
    if (int rc = element_bytes(t->dtype, eb)) return rc;
    const uint64_t start = t->off * eb;
    if (offset > ext - start || len > ext - start - offset) return err("tensor read outside extent");
    if (len && !out) return err("null output");
    FILE* f = fopen(p->data_path.c_str(), "rb");
    if (!f) return err("cannot open " + p->data_path);
    const bool ok = fseeko(f, (off_t)(p->storages[t->storage].offset + start + offset), SEEK_SET) == 0 &&
                    fread(out, 1, len, f) == len;
    fclose(f);
    return ok ? 0 : err("short read of " + p->data_path);
}

// Prepared::load_selected (prepared.rs:270-366): the storages holding a tensor under one of the prefixes (all when
// there are none) are allocated (device storages with hipMalloc, host ones in memory), then data.bin is read chunk by
// chunk through pinned staging; every chunk that overlaps a selected storage is SHA-256-checked against the manifest
// before its bytes are copied (the chunks of a batch are hashed in parallel threads, which the reference does one at
// a time). Requires 8 GiB of device memory to stay free, as the reference does.
int gfr_prepared_load(gfr_prepared* p, const char* const* prefixes, int nprefixes) {
    if (!p || nprefixes < 0 || (nprefixes && !prefixes)) return err("bad arguments");
    release(p);
    std::vector<bool> sel(p->storages.size(), nprefixes == 0);
    for (auto& kv : p->tensors)
        for (int i = 0; i < nprefixes; ++i)
            if (prefixes[i] && kv.first.compare(0, strlen(prefixes[i]), prefixes[i]) == 0) sel[kv.second.storage] = true;
    uint64_t bytes = 0;
    for (size_t j = 0; j < p->storages.size(); ++j)
        if (sel[j] && p->storages[j].cuda) bytes += p->storages[j].nbytes;
    size_t free_b = 0, total_b = 0;
    hipError_t e = hipMemGetInfo(&free_b, &total_b);
    if (e != hipSuccess) return gfr::set_error((int)e, std::string("hipMemGetInfo: ") + hipGetErrorString(e));
    if (bytes + (8ull << 30) >= (uint64_t)free_b) return err("not enough memory with 8 GiB reserve");
    const auto t0 = std::chrono::steady_clock::now();
    for (size_t j = 0; j < p->storages.size(); ++j) {
        if (!sel[j]) continue;
        if (p->storages[j].cuda) {
            if ((e = hipMalloc(&p->dev[j], p->storages[j].nbytes)) != hipSuccess) {
                p->dev[j] = nullptr;
                release(p);
                return gfr::set_error((int)e, std::string("hipMalloc: ") + hipGetErrorString(e));
            }
        } else {
            p->host[j].resize(p->storages[j].nbytes);
        }
    }
    // staging: a ring of pinned chunk slots (at most 1 GiB). Each needed chunk is read (pread at its offset) and
    // hashed in a task of its own; the oldest is checked and copied out when the ring is full, so up to 2 * 16 reads
    // and hashes and the copies overlap.
    const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const uint64_t nslot = std::max<uint64_t>(1, std::min<uint64_t>(2 * hw, (1ull << 30) / p->chunk));
    uint8_t* staging = nullptr;
    if ((e = hipHostMalloc((void**)&staging, nslot * p->chunk, hipHostMallocDefault)) != hipSuccess) {
        release(p);
        return gfr::set_error((int)e, std::string("hipHostMalloc: ") + hipGetErrorString(e));
    }
    const int fd = open(p->data_path.c_str(), O_RDONLY);
    int rc = fd >= 0 ? 0 : err("cannot open " + p->data_path);
    size_t first = 0;
    auto needed = [&](uint64_t off, uint64_t len) {
        for (size_t j = 0; j < p->storages.size(); ++j)
            if (sel[j] && p->storages[j].offset < off + len && p->storages[j].offset + p->storages[j].nbytes > off)
                return true;
        return false;
    };
    struct Pending {
        size_t chunk;
        uint8_t* data;
        std::future<std::string> hash;
    };
    std::deque<Pending> q;
    // the oldest read chunk: its hash checked, then its bytes copied into the storages it overlaps
    auto retire = [&]() -> int {
        Pending pd = std::move(q.front());
        q.pop_front();
        const std::string got = pd.hash.get();
        const size_t i = pd.chunk;
        if (got.size() != 64) return err(got);       // the task's read failed
        if (got != p->chunk_sha256[i]) return err("weight hash mismatch in chunk " + std::to_string(i));
        const uint64_t offset = i * p->chunk, len = std::min(p->file_size - offset, p->chunk);
        while (first < p->storages.size() && p->storages[first].offset + p->storages[first].nbytes <= offset) ++first;
        for (size_t j = first; j < p->storages.size(); ++j) {
            const Storage& s = p->storages[j];
            if (s.offset >= offset + len) break;
            if (!sel[j]) continue;
            const uint64_t lo = std::max(s.offset, offset), hi = std::min(s.offset + s.nbytes, offset + len);
            if (hi <= lo) continue;
            const uint8_t* src = pd.data + (lo - offset);
            if (s.cuda) {
                const hipError_t ce = hipMemcpy((uint8_t*)p->dev[j] + (lo - s.offset), src, hi - lo, hipMemcpyHostToDevice);
                if (ce != hipSuccess) return gfr::set_error((int)ce, std::string("hipMemcpy: ") + hipGetErrorString(ce));
            } else {
                memcpy(p->host[j].data() + (lo - s.offset), src, hi - lo);
            }
        }
        return 0;
    };
    uint64_t nread = 0;
    for (size_t i = 0; rc == 0 && i < p->chunk_sha256.size(); ++i) {
        const uint64_t off = i * p->chunk, len = std::min(p->file_size - off, p->chunk);
        if (!needed(off, len)) continue;
        if (q.size() == nslot && (rc = retire())) break;   // slots are freed oldest first: the ring stays in order
        uint8_t* buf = staging + (nread++ % nslot) * p->chunk;
        const std::string path = p->data_path;
        q.push_back({i, buf, std::async(std::launch::async, [buf, len, off, fd, path] {
                         for (uint64_t done = 0; done < len;) {
                             const ssize_t r = pread(fd, buf + done, len - done, (off_t)(off + done));
                             if (r <= 0) return std::string("short read of ") + path;
                             done += (uint64_t)r;
                         }
                         Sha256 h;
                         h.update(buf, len);
                         return h.hex();
                     })});
    }
    while (!q.empty()) {                        // every hash task is joined, also after an error
        if (rc) { q.front().hash.wait(); q.pop_front(); continue; }
        rc = retire();
    }
    if (fd >= 0) close(fd);
    (void)hipHostFree(staging);
    if (rc == 0 && (e = hipDeviceSynchronize()) != hipSuccess)
        rc = gfr::set_error((int)e, std::string("hipDeviceSynchronize: ") + hipGetErrorString(e));
    if (rc) { release(p); return rc; }
    for (size_t j = 0; j < p->storages.size(); ++j) p->loaded[j] = sel[j];
    p->loaded_bytes = bytes;
    p->load_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return 0;
}

int gfr_prepared_loaded(const gfr_prepared* p, uint64_t* bytes, double* seconds) {
    if (!p) return err("null prepared");
    if (bytes) *bytes = p->loaded_bytes;
    if (seconds) *seconds = p->load_seconds;
    return 0;
}

// Loaded::pointer (prepared.rs:369-377)
int gfr_prepared_pointer(const gfr_prepared* p, const char* path, void** ptr) {
    const Tensor* t = find(p, path);
    if (!t) return err(std::string("missing tensor ") + (path ? path : "(null)"));
    if (!ptr) return err("null output");
    *ptr = nullptr;
    if (!p->loaded[t->storage]) return err(std::string("tensor was not loaded: ") + path);
    if (!t->cuda) return err(std::string("CPU tensor has no GPU pointer: ") + path);
    uint64_t eb;
    if (int rc = element_bytes(t->dtype, eb)) return rc;
    *ptr = (uint8_t*)p->dev[t->storage] + t->off * eb;
    return 0;
}

// One layer's experts by name, as the reference resolves them (experts.rs:467: weights.layers[L].moe.experts.*),
// with the shapes of its probe (experts.rs:146-156) generalised: gt/ut [E][hidden/16][inter/16][8 bits] int32,
// dt [E][inter/16][hidden/16][8 bits], suh_g/suh_u/svh_d [E][hidden], suh_d/svh_g/svh_u [E][inter] float16.
int gfr_prepared_experts(const gfr_prepared* p, int layer, gfr_exl3_experts* out) {
    if (!p || !out || layer < 0) return err("bad arguments");
    const std::string stem = "weights.layers[" + std::to_string(layer) + "].moe.experts.";
    const Tensor* gt = find(p, (stem + "gt").c_str());
    if (!gt) return err("missing tensor " + stem + "gt");
    if (gt->shape.size() != 4 || gt->shape[3] % 8) return err("unsupported tensor " + stem + "gt");
    const uint64_t E = gt->shape[0], H = gt->shape[1] * 16, I = gt->shape[2] * 16, bits = gt->shape[3] / 8;
    if (bits < 2 || bits > 5 || E > (1u << 20) || H > (1u << 20) || I > (1u << 20))
        return err("unsupported expert geometry in " + stem + "gt");
    const struct { const char* name; const char* dtype; std::vector<uint64_t> shape; } want[] = {
        {"gt", "int32", {E, H / 16, I / 16, 8 * bits}}, {"ut", "int32", {E, H / 16, I / 16, 8 * bits}},
        {"dt", "int32", {E, I / 16, H / 16, 8 * bits}}, {"suh_g", "float16", {E, H}}, {"suh_u", "float16", {E, H}},
        {"suh_d", "float16", {E, I}}, {"svh_g", "float16", {E, I}}, {"svh_u", "float16", {E, I}},
        {"svh_d", "float16", {E, H}}};
    void* ptr[9];
    for (int i = 0; i < 9; ++i) {
        const std::string path = stem + want[i].name;
        if (int rc = gfr_prepared_expect(p, path.c_str(), want[i].dtype, want[i].shape.data(), (int)want[i].shape.size()))
            return rc;
        if (int rc = gfr_prepared_pointer(p, path.c_str(), &ptr[i])) return rc;
    }
    *out = gfr_exl3_experts{(int)E, (int)H, (int)I, (int)bits, (const uint32_t*)ptr[0], (const uint32_t*)ptr[1],
                            (const uint32_t*)ptr[2], (const uint16_t*)ptr[3], (const uint16_t*)ptr[4],
                            (const uint16_t*)ptr[5], (const uint16_t*)ptr[6], (const uint16_t*)ptr[7],
                            (const uint16_t*)ptr[8]};
    return 0;
}

int gfr_prepared_shared_fp8(const gfr_prepared* p, int layer, gfr_fp8_shared_weights* out) {
    if (!p || !out || layer < 0) return err("bad arguments");
    const std::string stem = "weights.layers[" + std::to_string(layer) + "].moe.shared.";
    const Tensor* gu = find(p, (stem + "gu.weight").c_str());
    if (!gu) return err("missing tensor " + stem + "gu.weight");
    if (gu->shape.size() != 2 || gu->shape[0] % 2 || gu->shape[0] > (2u << 20) || gu->shape[1] > (1u << 20))
        return err("unsupported tensor " + stem + "gu.weight");
    const uint64_t I = gu->shape[0] / 2, H = gu->shape[1];
    const struct { const char* name; const char* dtype; std::vector<uint64_t> shape; } want[] = {
        {"gu.weight", "float8_e4m3fn", {2 * I, H}}, {"gu.scale", "bfloat16", {2 * I}},
        {"down.weight", "float8_e4m3fn", {H, I}}, {"down.scale", "bfloat16", {H}}};
    void* ptr[4];
    for (int i = 0; i < 4; ++i) {
        const std::string path = stem + want[i].name;
        if (int rc = gfr_prepared_expect(p, path.c_str(), want[i].dtype, want[i].shape.data(), (int)want[i].shape.size()))
            return rc;
        if (int rc = gfr_prepared_pointer(p, path.c_str(), &ptr[i])) return rc;
    }
    *out = gfr_fp8_shared_weights{(int)H, (int)I, (const uint8_t*)ptr[0], (const uint16_t*)ptr[1],
                                  (const uint8_t*)ptr[2], (const uint16_t*)ptr[3], nullptr, nullptr};
    return 0;
}

int gfr_prepared_destroy(gfr_prepared* p) {
    if (!p) return 0;
    release(p);
    delete p;
    return 0;
}

}  // extern "C"
