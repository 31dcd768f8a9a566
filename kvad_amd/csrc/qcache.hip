// The quantised-weight cache file ("NANOQ") read straight into device
// weights: the container is mapped and parsed once; an array moves to HBM in
// chunks read from the file (page cache) into pinned staging buffers by
// several threads at once, two buffers in turn, so reading a chunk overlaps
// the DMA of the one before.  Reading with pread, not through the mapping,
// takes no page fault per 4 KiB page.
//
// Reference: crates/llm/src/qcache.rs -- the format (:30-40, MAGIC and
// ALIGN :90-93), Container::open (:863-883) and slice (:906-911),
// parse_entry (:817-834), Mapped::build (:689-713) and vector (:781-790);
// the GPU backend's GGML entries in the same container
// (crates/gpu/src/qcache.rs:278-296, kind names crates/gpu/src/common.rs:1012-1019).
//
// Entries:
//   kvad "q8"  {scales: f32 span, qs: i8 span}   -> KH_Q8 as stored
//   kvad "q4"  {scales: f32 span, qs: u8 span}   -> KH_Q4 as stored
//   "f32"      {data: f32 span}                  -> KH_F32
//   GGML "q4k" {data: byte span of block_q4_K}   -> KH_Q4K as stored
//   GGML "q8"  {data: block_q8_0 bytes}          -> KH_Q8: scale = (f32)d, codes as stored
//   GGML "q4"  {data: block_q4_0 bytes}          -> KH_Q4: scale = (f32)d, nibbles as stored
// A span is [byte offset, element count].  GGML's Q8_0 and Q4_0 blocks hold
// the same codes as kvad's q8/q4 with an f16 scale, and f16 -> f32 is exact,
// so the repacked weight computes what the block computes; Q4_0's nibble
// order (byte j: element j low, j + 16 high) is kvad q4's (quant.rs:258-274).
// Provenance (version, sources, spec) is the caller's check on the header
// text, as Mapped::open (qcache.rs:620-668) does it.
#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

namespace kh {
namespace {

const unsigned char MAGIC[8] = {'N', 'A', 'N', 'O', 'Q', 0, 0, 1};
constexpr size_t ALIGN = 64;

// ---- a small JSON reader: enough for any header (unknown values are kept
// as parsed trees and ignored) -------------------------------------------------
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    unsigned long long u = 0;  // exact value of a non-negative integer literal
    bool is_uint = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json *get(const std::string &k) const {
        if (kind != OBJ) return nullptr;
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct Parser {
    const char *p, *end;
    std::string err;
    int depth = 0;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail_at(const char *what) {
        if (err.empty()) err = what;
        return false;
    }
    bool lit(const char *s) {
        size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return fail_at("bad literal");
        p += n;
        return true;
    }
    static void utf8(std::string &o, unsigned c) {
        if (c < 0x80) {
            o += (char)c;
        } else if (c < 0x800) {
            o += (char)(0xC0 | (c >> 6)), o += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += (char)(0xE0 | (c >> 12)), o += (char)(0x80 | ((c >> 6) & 0x3F)), o += (char)(0x80 | (c & 0x3F));
        } else {
            o += (char)(0xF0 | (c >> 18)), o += (char)(0x80 | ((c >> 12) & 0x3F));
            o += (char)(0x80 | ((c >> 6) & 0x3F)), o += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(unsigned &v) {
        if (end - p < 4) return fail_at("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail_at("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &o) {
        if (p >= end || *p != '"') return fail_at("expected a string");
        p++;
        while (p < end && *p != '"') {
            char c = *p++;
            if ((unsigned char)c < 0x20) return fail_at("control character in a string");
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p >= end) return fail_at("unterminated escape");
            char e = *p++;
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    unsigned v;
                    if (!hex4(v)) return false;
                    if (v >= 0xD800 && v < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        unsigned lo;
                        if (!hex4(lo)) return false;
                        v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(o, v);
                    break;
                }
                default: return fail_at("bad escape");
            }
        }
        if (p >= end) return fail_at("unterminated string");
        p++;
        return true;
    }
    bool number(Json &v) {
        const char *s = p;
        if (p < end && *p == '-') p++;
        bool frac = false;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
            if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
            p++;
        }
        std::string t(s, p);
        if (t.empty() || t == "-") return fail_at("bad number");
        char *e = nullptr;
        v.kind = Json::NUM;
        v.num = strtod(t.c_str(), &e);
        if (*e) return fail_at("bad number");
        if (!frac && t[0] != '-') {
            errno = 0;
            v.u = strtoull(t.c_str(), &e, 10);
            v.is_uint = errno == 0 && !*e;
        }
        return true;
    }
    bool value(Json &v) {
        if (++depth > 256) return fail_at("nested too deep");
        ws();
        if (p >= end) return fail_at("unexpected end");
        bool ok;
        switch (*p) {
            case '{': {
                p++;
                v.kind = Json::OBJ;
                ws();
                if (p < end && *p == '}') {
                    p++;
                    ok = true;
                    break;
                }
                for (;;) {
                    ws();
                    std::string k;
                    if (!string(k)) return false;
                    ws();
                    if (p >= end || *p != ':') return fail_at("expected ':'");
                    p++;
                    v.obj.emplace_back(std::move(k), Json{});
                    if (!value(v.obj.back().second)) return false;
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        p++;
                        break;
                    }
                    return fail_at("expected ',' or '}'");
                }
                ok = true;
                break;
            }
            case '[': {
                p++;
                v.kind = Json::ARR;
                ws();
                if (p < end && *p == ']') {
                    p++;
                    ok = true;
                    break;
                }
                for (;;) {
                    v.arr.emplace_back();
                    if (!value(v.arr.back())) return false;
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        p++;
                        break;
                    }
                    return fail_at("expected ',' or ']'");
                }
                ok = true;
                break;
            }
            case '"': v.kind = Json::STR; ok = string(v.str); break;
            case 't': v.kind = Json::BOOL; v.b = true; ok = lit("true"); break;
            case 'f': v.kind = Json::BOOL; ok = lit("false"); break;
            case 'n': ok = lit("null"); break;
            default: ok = number(v); break;
        }
        depth--;
        return ok;
    }
};

// ---- entries -------------------------------------------------------------------
enum Layout { KVAD_SOA, F32_DATA, GGML_Q4K, GGML_Q8_0, GGML_Q4_0 };

struct Span {
    size_t off = 0, count = 0;
};

struct Entry {
    Layout layout;
    int precision;  // what the device weight will be
    size_t rows, cols;
    Span a, b;  // SoA: a = scales (f32), b = qs (i8/u8); otherwise a = data
};

}  // namespace
}  // namespace kh

struct kh_qcache {
    int fd = -1;
    const unsigned char *map = nullptr;
    size_t size = 0;
    std::string header;
    std::vector<std::string> names;  // in header order
    std::map<std::string, kh::Entry> entries;
    void *pin[2] = {nullptr, nullptr};  // pinned staging, made on the first upload
    std::mutex mu;                      // one upload at a time per handle (the staging is shared)
    ~kh_qcache() {
        for (void *p : pin)
            if (p) (void)hipHostFree(p);
        if (map) munmap(const_cast<unsigned char *>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace kh {
namespace {

bool span_of(const Json &e, const char *key, Span &s) {
    const Json *a = e.get(key);
    if (!a || a->kind != Json::ARR || a->arr.size() != 2 || !a->arr[0].is_uint || !a->arr[1].is_uint) return false;
    s.off = (size_t)a->arr[0].u;
    s.count = (size_t)a->arr[1].u;
    return true;
}

// Container::slice (qcache.rs:906-911): a span must lie inside the file.
bool inside(const kh_qcache &qc, const Span &s, size_t elem) {
    if (s.count > (SIZE_MAX - s.off) / (elem ? elem : 1)) return false;
    const size_t len = s.count * elem;
    return s.off <= qc.size && len <= qc.size - s.off;
}

int parse_entry(const kh_qcache &qc, const std::string &name, const Json &e, Entry &out) {
    auto bad = [&](const std::string &why) { return fail(KH_EINVAL, "qcache: `" + name + "`: " + why); };
    const Json *kind = e.get("kind");
    const Json *shape = e.get("shape");
    if (!kind || kind->kind != Json::STR) return bad("no `kind`");
    if (!shape || shape->kind != Json::ARR || shape->arr.size() != 2 || !shape->arr[0].is_uint ||
        !shape->arr[1].is_uint)
        return bad("no `shape`");
    out.rows = (size_t)shape->arr[0].u;
    out.cols = (size_t)shape->arr[1].u;
    if (out.rows == 0 || out.cols == 0 || out.rows > (size_t)INT32_MAX || out.cols > (size_t)INT32_MAX)
        return bad("bad shape");
    const size_t n = out.rows * out.cols;
    const std::string &k = kind->str;
    const bool soa = e.get("scales") && e.get("qs");
    if ((k == "q8" || k == "q4") && soa) {
        out.layout = KVAD_SOA;
        out.precision = k == "q8" ? KH_Q8 : KH_Q4;
        if (!span_of(e, "scales", out.a) || !span_of(e, "qs", out.b)) return bad("bad span");
        if (out.cols % BLOCK) return bad("cols is not a multiple of 32");
        if (out.a.count != n / BLOCK || out.b.count != (k == "q8" ? n : n / 2)) return bad("span length does not match shape");
        if (!inside(qc, out.a, 4) || !inside(qc, out.b, 1)) return bad("array runs past the end of the file");
        return KH_OK;
    }
    if (!span_of(e, "data", out.a)) return bad("bad span");
    if (k == "f32") {
        out.layout = F32_DATA;
        out.precision = KH_F32;
        if (out.a.count != n) return bad("span length does not match shape");
        if (!inside(qc, out.a, 4)) return bad("array runs past the end of the file");
        return KH_OK;
    }
    size_t bpb, per;  // bytes per block, weights per block
    if (k == "q4k") out.layout = GGML_Q4K, out.precision = KH_Q4K, bpb = Q4K_BYTES, per = QK_K;
    else if (k == "q8") out.layout = GGML_Q8_0, out.precision = KH_Q8, bpb = 34, per = BLOCK;
    else if (k == "q4") out.layout = GGML_Q4_0, out.precision = KH_Q4, bpb = 18, per = BLOCK;
    else return fail(KH_DECLINED, "qcache: `" + name + "`: kind `" + k + "` has no device kernel here");
    if (out.cols % per) return bad("cols is not a multiple of the block");
    if (out.a.count != n / per * bpb) return bad("span length does not match shape");
    if (!inside(qc, out.a, 1)) return bad("array runs past the end of the file");
    return KH_OK;
}

// ---- host -> device through pinned staging ---------------------------------------
constexpr size_t CHUNK = 32u << 20;
constexpr int READERS = 4;  // threads reading one chunk from the file

// Reads n bytes at file offset off into dst with READERS threads; false on a
// short read.
bool read_at(int fd, unsigned char *dst, size_t n, size_t off) {
    bool ok[READERS];
    auto part = [&](int t) {
        const size_t a = n * t / READERS, b = n * (t + 1) / READERS;
        ok[t] = true;
        for (size_t at = a; at < b;) {
            const ssize_t r = pread(fd, dst + at, b - at, (off_t)(off + at));
            if (r <= 0) {
                if (r < 0 && errno == EINTR) continue;
                ok[t] = false;
                return;
            }
            at += (size_t)r;
        }
    };
    if (n < (1u << 20)) {
        for (int t = 0; t < READERS; t++) part(t);
    } else {
        std::thread th[READERS - 1];
        for (int t = 1; t < READERS; t++) th[t - 1] = std::thread(part, t);
        part(0);
        for (auto &x : th) x.join();
    }
    for (bool o : ok)
        if (!o) return false;
    return true;
}

struct Stager {
    kh_ctx *ctx;
    kh_qcache *qc;
    hipEvent_t done[2] = {nullptr, nullptr};
    int next = 0;
    ~Stager() {
        if (ctx) (void)hipStreamSynchronize(ctx->stream);
        for (auto &e : done)
            if (e) (void)hipEventDestroy(e);
    }
    int init() {
        for (int i = 0; i < 2; i++) {
            if (!qc->pin[i]) KH_HIP(hipHostMalloc(&qc->pin[i], CHUNK, hipHostMallocDefault));
            KH_HIP(hipEventCreateWithFlags(&done[i], hipEventDisableTiming));
            KH_HIP(hipEventRecord(done[i], ctx->stream));
        }
        return KH_OK;
    }
    // `fill(buf, first, n)` writes bytes [first, first + n) of the array into
    // the staging buffer buf, which the copy that last used it has finished with.
    template <typename F>
    int copy(void *dst, size_t bytes, F fill) {
        for (size_t at = 0; at < bytes; at += CHUNK) {
            const size_t n = bytes - at < CHUNK ? bytes - at : CHUNK;
            KH_HIP(hipEventSynchronize(done[next]));
            unsigned char *buf = static_cast<unsigned char *>(qc->pin[next]);
            if (!fill(buf, at, n)) return fail(KH_EINVAL, "qcache: short read from the file");
            KH_HIP(hipMemcpyAsync(static_cast<unsigned char *>(dst) + at, buf, n, hipMemcpyHostToDevice, ctx->stream));
            KH_HIP(hipEventRecord(done[next], ctx->stream));
            next ^= 1;
        }
        return KH_OK;
    }
    // A span of the file, as it lies.
    int file(void *dst, size_t bytes, size_t off) {
        return copy(dst, bytes, [&](unsigned char *b, size_t at, size_t n) { return read_at(qc->fd, b, n, off + at); });
    }
};

float half_to_float(const unsigned char *p) {
    unsigned short h;
    memcpy(&h, p, 2);
    return (float)__builtin_bit_cast(_Float16, h);
}

}  // namespace
}  // namespace kh

using namespace kh;

extern "C" {

int kh_qcache_open(const char *path, kh_qcache **out) {
    if (!path || !out) return fail(KH_EINVAL, "kh_qcache_open: null argument");
    *out = nullptr;
    std::unique_ptr<kh_qcache> qc(new kh_qcache());
    qc->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (qc->fd < 0) return fail(KH_EINVAL, std::string("kh_qcache_open: cannot open ") + path);
    struct stat st;
    if (fstat(qc->fd, &st) != 0) return fail(KH_EINVAL, "kh_qcache_open: cannot stat the file");
    qc->size = (size_t)st.st_size;
    if (qc->size < ALIGN + 8) return fail(KH_EINVAL, "kh_qcache_open: not a quantised-weight file");
    void *m = mmap(nullptr, qc->size, PROT_READ, MAP_PRIVATE, qc->fd, 0);
    if (m == MAP_FAILED) return fail(KH_EINVAL, "kh_qcache_open: cannot map the file");
    qc->map = static_cast<const unsigned char *>(m);
    if (memcmp(qc->map, MAGIC, 8) != 0) return fail(KH_EINVAL, "kh_qcache_open: not a quantised-weight file");
    // the header sits just before the trailing u64, which says where it starts
    unsigned long long at;
    memcpy(&at, qc->map + qc->size - 8, 8);
    if (at < ALIGN || at > qc->size - 8) return fail(KH_EINVAL, "kh_qcache_open: header offset is out of range");
    qc->header.assign(reinterpret_cast<const char *>(qc->map + at), qc->size - 8 - (size_t)at);
    Json root;
    Parser ps{qc->header.data(), qc->header.data() + qc->header.size()};
    if (!ps.value(root)) return fail(KH_EINVAL, "kh_qcache_open: header is not JSON (" + ps.err + ")");
    ps.ws();
    if (ps.p != ps.end) return fail(KH_EINVAL, "kh_qcache_open: trailing bytes after the header");
    const Json *tensors = root.get("tensors");
    if (tensors && tensors->kind != Json::OBJ) return fail(KH_EINVAL, "kh_qcache_open: `tensors` is not an object");
    if (tensors) {
        for (auto &kv : tensors->obj) {
            Entry e;
            if (kv.second.kind != Json::OBJ) return fail(KH_EINVAL, "qcache: `" + kv.first + "` is not an object");
            int rc = parse_entry(*qc, kv.first, kv.second, e);
            if (rc == KH_DECLINED) continue;  // kept out of the table: the caller quantises it itself
            if (rc) return rc;
            if (qc->entries.emplace(kv.first, e).second) qc->names.push_back(kv.first);
        }
    }
    *out = qc.release();
    return KH_OK;
}

int kh_qcache_free(kh_qcache *qc) {
    delete qc;
    return KH_OK;
}

const char *kh_qcache_header(const kh_qcache *qc) { return qc ? qc->header.c_str() : nullptr; }

int kh_qcache_count(const kh_qcache *qc, size_t *n) {
    if (!qc || !n) return fail(KH_EINVAL, "kh_qcache_count: null argument");
    *n = qc->names.size();
    return KH_OK;
}

const char *kh_qcache_name(const kh_qcache *qc, size_t i) {
    if (!qc || i >= qc->names.size()) return nullptr;
    return qc->names[i].c_str();
}

int kh_qcache_info(const kh_qcache *qc, const char *name, int *precision, size_t *rows, size_t *cols) {
    if (!qc || !name) return fail(KH_EINVAL, "kh_qcache_info: null argument");
    auto it = qc->entries.find(name);
    if (it == qc->entries.end()) return fail(KH_EINVAL, std::string("qcache: no tensor `") + name + "`");
    if (precision) *precision = it->second.precision;
    if (rows) *rows = it->second.rows;
    if (cols) *cols = it->second.cols;
    return KH_OK;
}

int kh_qcache_vector(const kh_qcache *qc, const char *name, float *out, size_t n) {
    if (!qc || !name || (!out && n)) return fail(KH_EINVAL, "kh_qcache_vector: null argument");
    auto it = qc->entries.find(name);
    if (it == qc->entries.end()) return fail(KH_EINVAL, std::string("qcache: no tensor `") + name + "`");
    const Entry &e = it->second;
    if (e.layout != F32_DATA || e.rows != 1) return fail(KH_EINVAL, std::string("qcache: `") + name + "` is not a vector");
    if (n != e.cols) return fail(KH_EINVAL, std::string("qcache: `") + name + "` holds " + std::to_string(e.cols) + " values");
    memcpy(out, qc->map + e.a.off, 4 * n);
    return KH_OK;
}

int kh_qcache_weight(kh_ctx *ctx, const kh_qcache *cqc, const char *name, kh_weight **out) {
    kh_qcache *qc = const_cast<kh_qcache *>(cqc);  // the staging buffers are the handle's
    if (!ctx || !qc || !name || !out) return fail(KH_EINVAL, "kh_qcache_weight: null argument");
    *out = nullptr;
    auto it = qc->entries.find(name);
    if (it == qc->entries.end()) return fail(KH_EINVAL, std::string("qcache: no tensor `") + name + "`");
    const Entry &e = it->second;
    std::lock_guard<std::mutex> qlock(qc->mu);
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    std::unique_ptr<kh_weight> w(new kh_weight());
    w->ctx = ctx;
    w->precision = e.precision;
    w->rows = e.rows;
    w->cols = e.cols;
    const size_t n = e.rows * e.cols;
    size_t qs_bytes, n_scales = 0;
    switch (e.precision) {
        case KH_Q8: qs_bytes = n, n_scales = n / BLOCK; break;
        case KH_Q4: qs_bytes = n / 2, n_scales = n / BLOCK; break;
        case KH_Q4K: qs_bytes = n / QK_K * Q4K_BYTES; break;
        default: qs_bytes = 4 * n; break;
    }
    // hold the device arrays in the weight as soon as they exist, so an error
    // part-way frees them with it
    struct Owner {
        std::unique_ptr<kh_weight> &w;
        ~Owner() {
            if (w) {
                if (w->qs) (void)hipFree(w->qs);
                if (w->scales) (void)hipFree(w->scales);
            }
        }
    } own{w};
    KH_HIP(hipMalloc(&w->qs, qs_bytes));
    if (n_scales) KH_HIP(hipMalloc(reinterpret_cast<void **>(&w->scales), 4 * n_scales));
    Stager st{ctx, qc};
    int rc = st.init();
    if (rc) return rc;
    const unsigned char *base = qc->map;
    if (e.layout == KVAD_SOA) {
        if ((rc = st.file(w->qs, qs_bytes, e.b.off))) return rc;
        if ((rc = st.file(w->scales, 4 * n_scales, e.a.off))) return rc;
    } else if (e.layout == F32_DATA || e.layout == GGML_Q4K) {
        if ((rc = st.file(w->qs, qs_bytes, e.a.off))) return rc;
    } else {
        // GGML Q8_0 / Q4_0: [f16 d][codes] blocks -> codes and f32 scales
        const size_t bpb = e.layout == GGML_Q8_0 ? 34 : 18, cb = bpb - 2;  // code bytes per block
        const unsigned char *src = base + e.a.off;
        if ((rc = st.copy(w->qs, qs_bytes, [&](unsigned char *d, size_t at, size_t k) {
                 // bytes [at, at + k) of the codes: whole blocks, as CHUNK % cb == 0 for cb 32 and 16
                 for (size_t o = 0; o < k; o += cb) memcpy(d + o, src + (at + o) / cb * bpb + 2, cb);
                 return true;
             })))
            return rc;
        if ((rc = st.copy(w->scales, 4 * n_scales, [&](unsigned char *d, size_t at, size_t k) {
                 for (size_t o = 0; o < k; o += 4) {
                     const float s = half_to_float(src + (at + o) / 4 * bpb);
                     memcpy(d + o, &s, 4);
                 }
                 return true;
             })))
            return rc;
    }
    KH_HIP(hipStreamSynchronize(ctx->stream));
    w->bytes = qs_bytes + 4 * n_scales;
    *out = w.release();
    return KH_OK;
}

}  // extern "C"
