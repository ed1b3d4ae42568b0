// Weight files of the decoder LM runner: save / load / read_config.
//
// The reference has no on-disk weight format: its nets receive weights only through the
// init_weight<I>() traversal hook (mat_init_t.hpp:113-118, mat_net_t.hpp:51-56).  This
// build stores a runner's weights in the safetensors container, so that other tools can
// read and write them:
//   [8 bytes: header length N, little endian][N bytes: JSON header, space padded][data]
// The header maps each tensor name to {"dtype", "shape", "data_offsets": [begin, end)}
// (offsets relative to the start of the data), plus "__metadata__", a string -> string map
// that holds the runner's config.  Tensors use the names and the logical row-major order
// of jas_lm_get_weight / jas_lm_set_weight, with shape [layers, rows, cols].  F32 and BF16
// data are accepted on load; save writes BF16 for tensors stored as bf16, F32 otherwise.
//
// Loading streams the file through two pinned staging buffers: while the device copies
// one chunk, the host reads the next.  A projection matrix is packed into the MFMA-native
// layout on the device, one layer at a time, from its logical form.
#include "lm.hpp"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

namespace jas {
namespace {

// ------------------------------------------------------------------ JSON (header only)
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    bool integral = false;
    long long i = 0;
    double d = 0;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal *get(const std::string &k) const
    {
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char *p, *end;
    std::string err;
    int depth = 0;

    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char *m)
    {
        if (err.empty()) err = m;
        return false;
    }
    static void utf8(std::string &o, unsigned cp)
    {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | cp >> 6); o += (char)(0x80 | (cp & 63)); }
        else if (cp < 0x10000) { o += (char)(0xE0 | cp >> 12); o += (char)(0x80 | (cp >> 6 & 63)); o += (char)(0x80 | (cp & 63)); }
        else { o += (char)(0xF0 | cp >> 18); o += (char)(0x80 | (cp >> 12 & 63)); o += (char)(0x80 | (cp >> 6 & 63)); o += (char)(0x80 | (cp & 63)); }
    }
    bool hex4(unsigned &v)
    {
        if (end - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string &o)
    {
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        while (p < end && *p != '"') {
            if ((unsigned char)*p < 0x20) return fail("control character in a string");
            if (*p != '\\') { o += *p++; continue; }
            if (++p >= end) break;
            const char c = *p++;
            switch (c) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                unsigned cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                    p += 2;
                    unsigned lo;
                    if (!hex4(lo)) return false;
                    if (lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(o, cp);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool num(JVal &v)
    {
        const char *b = p;
        if (p < end && *p == '-') ++p;
        while (p < end && *p >= '0' && *p <= '9') ++p;
        bool integral = true;
        if (p < end && *p == '.') { integral = false; ++p; while (p < end && *p >= '0' && *p <= '9') ++p; }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        if (p == b || (p == b + 1 && *b == '-')) return fail("bad number");
        const std::string t(b, p);
        v.kind = JVal::Num;
        v.integral = integral;
        errno = 0;
        if (integral) {
            v.i = strtoll(t.c_str(), nullptr, 10);
            if (errno == ERANGE) return fail("integer out of range");
            v.d = (double)v.i;
        } else {
            v.d = strtod(t.c_str(), nullptr);
        }
        return true;
    }
    bool lit(const char *w)
    {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return fail("bad literal");
        p += n;
        return true;
    }
    bool value(JVal &v)
    {
        if (++depth > 32) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end of header");
        bool ok = true;
        if (*p == '{') {
            v.kind = JVal::Obj;
            ++p;
            ws();
            if (p < end && *p == '}') ++p;
            else
                for (;;) {
                    std::pair<std::string, JVal> kv;
                    ws();
                    if (!str(kv.first)) { ok = false; break; }
                    ws();
                    if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
                    ++p;
                    if (!value(kv.second)) { ok = false; break; }
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == '}') { ++p; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
        } else if (*p == '[') {
            v.kind = JVal::Arr;
            ++p;
            ws();
            if (p < end && *p == ']') ++p;
            else
                for (;;) {
                    JVal e;
                    if (!value(e)) { ok = false; break; }
                    v.arr.push_back(std::move(e));
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == ']') { ++p; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
        } else if (*p == '"') {
            v.kind = JVal::Str;
            ok = str(v.s);
        } else if (*p == 't') {
            v.kind = JVal::Bool, v.b = true, ok = lit("true");
        } else if (*p == 'f') {
            v.kind = JVal::Bool, ok = lit("false");
        } else if (*p == 'n') {
            ok = lit("null");
        } else {
            ok = num(v);
        }
        --depth;
        return ok;
    }
};

std::string json_escape(const std::string &s)
{
    std::string o;
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') { o += '\\'; o += (char)c; }
        else if (c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
        else o += (char)c;
    }
    return o;
}

// ------------------------------------------------------------------ file header
struct FileTensor {
    std::string name;
    bool bf16 = false;       // element type in the file
    long layers = 1, rows = 1, cols = 1;
    unsigned long long begin = 0, end = 0;  // relative to the data section
};

struct FileHeader {
    std::vector<FileTensor> tensors;
    std::vector<std::pair<std::string, std::string>> meta;
    unsigned long long data_start = 0, data_bytes = 0;
    const FileTensor *find(const std::string &n) const
    {
        for (auto &t : tensors)
            if (t.name == n) return &t;
        return nullptr;
    }
    const std::string *meta_get(const std::string &k) const
    {
        for (auto &kv : meta)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

constexpr unsigned long long kMaxHeader = 100ull << 20;

struct File {
    int fd = -1;
    ~File()
    {
        if (fd >= 0) close(fd);
    }
};

// read exactly n bytes at offset off
bool read_at(int fd, void *dst, size_t n, unsigned long long off)
{
    char *d = (char *)dst;
    while (n) {
        const ssize_t r = pread(fd, d, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        d += r, n -= (size_t)r, off += (unsigned long long)r;
    }
    return true;
}

bool write_all(int fd, const void *src, size_t n)
{
    const char *s = (const char *)src;
    while (n) {
        const ssize_t r = write(fd, s, n);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        s += r, n -= (size_t)r;
    }
    return true;
}

jas_status parse_header(const char *path, File &f, FileHeader &h)
{
    const std::string where = std::string("jas_lm weight file ") + path + ": ";
    f.fd = open(path, O_RDONLY | O_CLOEXEC);
    JAS_CHECK(f.fd >= 0, JAS_ERR_RUNTIME, where + strerror(errno));
    struct stat st;
    JAS_CHECK(fstat(f.fd, &st) == 0, JAS_ERR_RUNTIME, where + strerror(errno));
    const unsigned long long fsize = (unsigned long long)st.st_size;
    unsigned char lb[8];
    JAS_CHECK(fsize >= 8 && read_at(f.fd, lb, 8, 0), JAS_ERR_INVALID, where + "shorter than the 8-byte header length");
    unsigned long long n = 0;
    for (int k = 7; k >= 0; --k) n = n << 8 | lb[k];
    JAS_CHECK(n >= 2 && n <= kMaxHeader && n <= fsize - 8, JAS_ERR_INVALID, where + "bad header length");
    std::string text(n, '\0');
    JAS_CHECK(read_at(f.fd, &text[0], n, 8), JAS_ERR_INVALID, where + "truncated header");
    JParser jp{text.data(), text.data() + text.size()};
    JVal root;
    const bool ok = jp.value(root);
    JAS_CHECK(ok, JAS_ERR_INVALID, where + "header is not valid JSON (" + jp.err + ")");
    jp.ws();
    JAS_CHECK(jp.p == jp.end, JAS_ERR_INVALID, where + "trailing bytes after the header object");
    JAS_CHECK(root.kind == JVal::Obj, JAS_ERR_INVALID, where + "header is not a JSON object");
    h.data_start = 8 + n;
    h.data_bytes = fsize - h.data_start;
    for (auto &kv : root.obj) {
        if (kv.first == "__metadata__") {
            JAS_CHECK(kv.second.kind == JVal::Obj, JAS_ERR_INVALID, where + "__metadata__ is not an object");
            for (auto &m : kv.second.obj) {
                JAS_CHECK(m.second.kind == JVal::Str, JAS_ERR_INVALID, where + "__metadata__ values must be strings");
                h.meta.emplace_back(m.first, m.second.s);
            }
            continue;
        }
        const JVal &e = kv.second;
        const std::string tw = where + "tensor '" + kv.first + "': ";
        JAS_CHECK(e.kind == JVal::Obj, JAS_ERR_INVALID, tw + "entry is not an object");
        const JVal *dt = e.get("dtype"), *sh = e.get("shape"), *of = e.get("data_offsets");
        JAS_CHECK(dt && dt->kind == JVal::Str && sh && sh->kind == JVal::Arr && of && of->kind == JVal::Arr,
                  JAS_ERR_INVALID, tw + "needs dtype, shape and data_offsets");
        FileTensor t;
        t.name = kv.first;
        JAS_CHECK(dt->s == "F32" || dt->s == "BF16", JAS_ERR_INVALID, tw + "dtype " + dt->s + " (F32 or BF16 expected)");
        t.bf16 = dt->s == "BF16";
        JAS_CHECK(sh->arr.size() >= 1 && sh->arr.size() <= 3, JAS_ERR_INVALID, tw + "shape must have 1 to 3 dimensions");
        long dims[3] = {1, 1, 1};
        const size_t r = sh->arr.size();
        for (size_t k = 0; k < r; ++k) {
            const JVal &d = sh->arr[k];
            JAS_CHECK(d.kind == JVal::Num && d.integral && d.i >= 0 && d.i <= INT32_MAX, JAS_ERR_INVALID,
                      tw + "bad shape entry");
            dims[3 - r + k] = (long)d.i;
        }
        t.layers = dims[0], t.rows = dims[1], t.cols = dims[2];
        JAS_CHECK(of->arr.size() == 2 && of->arr[0].kind == JVal::Num && of->arr[1].kind == JVal::Num &&
                      of->arr[0].integral && of->arr[1].integral && of->arr[0].i >= 0 && of->arr[1].i >= of->arr[0].i,
                  JAS_ERR_INVALID, tw + "bad data_offsets");
        t.begin = (unsigned long long)of->arr[0].i;
        t.end = (unsigned long long)of->arr[1].i;
        unsigned long long want = t.bf16 ? 2 : 4;
        const bool ovf = __builtin_mul_overflow(want, (unsigned long long)t.layers, &want) ||
                         __builtin_mul_overflow(want, (unsigned long long)t.rows, &want) ||
                         __builtin_mul_overflow(want, (unsigned long long)t.cols, &want);
        JAS_CHECK(!ovf && t.end - t.begin == want, JAS_ERR_INVALID, tw + "data_offsets do not match shape and dtype");
        JAS_CHECK(t.end <= h.data_bytes, JAS_ERR_INVALID, tw + "data runs past the end of the file");
        JAS_CHECK(!h.find(t.name), JAS_ERR_INVALID, tw + "listed twice");
        h.tensors.push_back(t);
    }
    return JAS_OK;
}

// ------------------------------------------------------------------ config <-> metadata
struct CfgField {
    const char *key;
    int32_t jas_lm_config::*i;
    float jas_lm_config::*f;
};
const CfgField kCfgFields[] = {
    {"kind", &jas_lm_config::kind, nullptr},
    {"n_layer", &jas_lm_config::n_layer, nullptr},
    {"d_model", &jas_lm_config::d_model, nullptr},
    {"n_head", &jas_lm_config::n_head, nullptr},
    {"d_ff", &jas_lm_config::d_ff, nullptr},
    {"vocab", &jas_lm_config::vocab, nullptr},
    {"max_ctx", &jas_lm_config::max_ctx, nullptr},
    {"max_batch", &jas_lm_config::max_batch, nullptr},
    {"eps", nullptr, &jas_lm_config::eps},
    {"rope_theta", nullptr, &jas_lm_config::rope_theta},
    {"weight_bf16", &jas_lm_config::weight_bf16, nullptr},
    {"kv_bf16", &jas_lm_config::kv_bf16, nullptr},
};
const char *kFormatKey = "format", *kFormatName = "jasmine_amd.lm";

// ------------------------------------------------------------------ device conversions
__global__ void widen_bf16_kernel(const uint16_t *__restrict__ src, float *__restrict__ dst, long n)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = bf16_to_f32(src[i]);
}

__global__ void narrow_bf16_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst, long n)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = f32_to_bf16(src[i]);
}

// Two pinned host buffers with an event each: the host fills / drains one while the device
// copies the other.
struct Staging {
    static constexpr size_t kChunk = 64u << 20;
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    int next = 0;
    ~Staging()
    {
        for (int k = 0; k < 2; ++k) {
            if (ev[k]) {
                (void)hipEventSynchronize(ev[k]);
                (void)hipEventDestroy(ev[k]);
            }
            if (buf[k]) (void)hipHostFree(buf[k]);
        }
    }
    jas_status init()
    {
        for (int k = 0; k < 2; ++k) {
            JAS_HIP(hipHostMalloc(&buf[k], kChunk, hipHostMallocDefault));
            JAS_HIP(hipEventCreateWithFlags(&ev[k], hipEventDisableTiming));
        }
        return JAS_OK;
    }
};

// file bytes [off, off + n) -> device dst, through the staging buffers
jas_status upload(int fd, unsigned long long off, size_t n, void *dst, Staging &sg, hipStream_t s, const std::string &what)
{
    char *d = (char *)dst;
    while (n) {
        const size_t c = n < Staging::kChunk ? n : Staging::kChunk;
        const int k = sg.next;
        sg.next ^= 1;
        JAS_HIP(hipEventSynchronize(sg.ev[k]));  // the copy out of this buffer has finished
        JAS_CHECK(read_at(fd, sg.buf[k], c, off), JAS_ERR_RUNTIME, what + ": read failed");
        JAS_HIP(hipMemcpyAsync(d, sg.buf[k], c, hipMemcpyHostToDevice, s));
        JAS_HIP(hipEventRecord(sg.ev[k], s));
        d += c, off += c, n -= c;
    }
    return JAS_OK;
}

// device src [0, n) -> file, through the staging buffers (the copy of one chunk overlaps
// the write of the previous one)
jas_status download(int fd, const void *src, size_t n, Staging &sg, hipStream_t s, const std::string &what)
{
    const char *p = (const char *)src;
    size_t pend[2] = {0, 0};
    auto drain = [&](int k) -> jas_status {
        if (!pend[k]) return JAS_OK;
        JAS_HIP(hipEventSynchronize(sg.ev[k]));
        JAS_CHECK(write_all(fd, sg.buf[k], pend[k]), JAS_ERR_RUNTIME, what + ": write failed");
        pend[k] = 0;
        return JAS_OK;
    };
    int k = 0;
    while (n) {
        const size_t c = n < Staging::kChunk ? n : Staging::kChunk;
        TRY(drain(k));
        JAS_HIP(hipMemcpyAsync(sg.buf[k], p, c, hipMemcpyDeviceToHost, s));
        JAS_HIP(hipEventRecord(sg.ev[k], s));
        pend[k] = c;
        k ^= 1;
        TRY(drain(k));  // the older chunk, in file order
        p += c, n -= c;
    }
    TRY(drain(k ^ 1));
    return drain(k);
}

struct DevBuf {
    void *p = nullptr;
    ~DevBuf()
    {
        if (p) (void)hipFree(p);
    }
};

} // namespace
} // namespace jas

using namespace jas;

extern "C" {

jas_status jas_lm_read_config(const char *path, jas_lm_config *cfg)
{
    JAS_CHECK(path && cfg, JAS_ERR_INVALID, "jas_lm_read_config: null argument");
    File f;
    FileHeader h;
    TRY(parse_header(path, f, h));
    const std::string *fmt = h.meta_get(kFormatKey);
    JAS_CHECK(fmt && *fmt == kFormatName, JAS_ERR_INVALID,
              std::string("jas_lm_read_config: ") + path + " carries no runner config (__metadata__ format != " +
                  kFormatName + ")");
    jas_lm_config c{};
    for (const CfgField &fd : kCfgFields) {
        const std::string *v = h.meta_get(fd.key);
        JAS_CHECK(v, JAS_ERR_INVALID, std::string("jas_lm_read_config: metadata lacks ") + fd.key);
        char *e = nullptr;
        errno = 0;
        if (fd.i) {
            const long x = strtol(v->c_str(), &e, 10);
            JAS_CHECK(e && *e == 0 && !v->empty() && errno == 0 && x >= INT32_MIN && x <= INT32_MAX, JAS_ERR_INVALID,
                      std::string("jas_lm_read_config: bad integer for ") + fd.key);
            c.*(fd.i) = (int32_t)x;
        } else {
            const float x = strtof(v->c_str(), &e);
            JAS_CHECK(e && *e == 0 && !v->empty() && std::isfinite(x), JAS_ERR_INVALID,
                      std::string("jas_lm_read_config: bad number for ") + fd.key);
            c.*(fd.f) = x;
        }
    }
    *cfg = c;
    return JAS_OK;
}

jas_status jas_lm_save(jas_lm *lm, const char *path)
{
    JAS_CHECK(lm && path, JAS_ERR_INVALID, "jas_lm_save: null argument");
    hipStream_t s = lm->stream;
    // header: tensors in name order, each [layers, rows, cols]
    std::string hdr = "{\"__metadata__\":{\"" + std::string(kFormatKey) + "\":\"" + kFormatName + "\"";
    for (const CfgField &fd : kCfgFields) {
        char b[64];
        if (fd.i) snprintf(b, sizeof b, "%d", (int)(lm->cfg.*(fd.i)));
        else snprintf(b, sizeof b, "%.9g", (double)(lm->cfg.*(fd.f)));
        hdr += ",\"" + std::string(fd.key) + "\":\"" + b + "\"";
    }
    hdr += "}";
    unsigned long long off = 0;
    size_t max_layer = 0;  // elements of the largest packed layer
    for (auto &kv : lm->tensors) {
        const Tensor &t = kv.second;
        if (t.count == 0) continue;
        const unsigned long long nb = (unsigned long long)t.layers * t.rows * t.cols * (t.bf16 ? 2 : 4);
        char b[256];
        snprintf(b, sizeof b, ",\"%s\":{\"dtype\":\"%s\",\"shape\":[%d,%d,%d],\"data_offsets\":[%llu,%llu]}",
                 json_escape(kv.first).c_str(), t.bf16 ? "BF16" : "F32", t.layers, t.rows, t.cols, off, off + nb);
        hdr += b;
        off += nb;
        if (t.packed) max_layer = std::max(max_layer, (size_t)t.rows * t.cols);
    }
    hdr += "}";
    while ((8 + hdr.size()) % 8) hdr += ' ';

    DevBuf tmp, narrow;
    if (max_layer) {
        JAS_HIP(hipMalloc(&tmp.p, max_layer * sizeof(float)));
        JAS_HIP(hipMalloc(&narrow.p, max_layer * sizeof(uint16_t)));
    }
    Staging sg;
    TRY(sg.init());
    const std::string tmp_path = std::string(path) + ".partial";
    File f;
    f.fd = open(tmp_path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    JAS_CHECK(f.fd >= 0, JAS_ERR_RUNTIME, std::string("jas_lm_save: ") + tmp_path + ": " + strerror(errno));
    unsigned char lb[8];
    unsigned long long n = hdr.size();
    for (int k = 0; k < 8; ++k) lb[k] = (unsigned char)(n >> (8 * k));
    jas_status st = JAS_OK;
    auto run = [&]() -> jas_status {
        JAS_CHECK(write_all(f.fd, lb, 8) && write_all(f.fd, hdr.data(), hdr.size()), JAS_ERR_RUNTIME,
                  "jas_lm_save: write failed");
        for (auto &kv : lm->tensors) {
            const Tensor &t = kv.second;
            if (t.count == 0) continue;
            const std::string what = "jas_lm_save: " + kv.first;
            const float *dev = lm->arena + t.off;
            if (!t.packed) {
                TRY(download(f.fd, dev, (size_t)t.layers * t.rows * t.cols * sizeof(float), sg, s, what));
                continue;
            }
            const long ne = (long)t.rows * t.cols;
            for (int l = 0; l < t.layers; ++l) {
                TRY(weight_pack(dev + l * t.lstride(), tmp.p, t.rows, t.cols, true, s, t.bf16));
                if (t.bf16) {
                    hipLaunchKernelGGL(narrow_bf16_kernel, dim3(ceil_div(ne, 256)), dim3(256), 0, s,
                                       (const float *)tmp.p, (uint16_t *)narrow.p, ne);
                    TRY(download(f.fd, narrow.p, ne * sizeof(uint16_t), sg, s, what));
                } else {
                    TRY(download(f.fd, tmp.p, ne * sizeof(float), sg, s, what));
                }
            }
        }
        JAS_HIP(hipStreamSynchronize(s));
        return JAS_OK;
    };
    st = run();
    if (close(f.fd) != 0 && st == JAS_OK) st = fail(JAS_ERR_RUNTIME, "jas_lm_save: close failed");
    f.fd = -1;
    if (st == JAS_OK && rename(tmp_path.c_str(), path) != 0)
        st = fail(JAS_ERR_RUNTIME, std::string("jas_lm_save: rename to ") + path + ": " + strerror(errno));
    if (st != JAS_OK) unlink(tmp_path.c_str());
    return st;
}

jas_status jas_lm_load(jas_lm *lm, const char *path)
{
    JAS_CHECK(lm && path, JAS_ERR_INVALID, "jas_lm_load: null argument");
    File f;
    FileHeader h;
    TRY(parse_header(path, f, h));
    hipStream_t s = lm->stream;
    // every tensor of the model must be in the file with its shape, and nothing else;
    // a learned position table may hold more positions than max_ctx (its prefix is used)
    size_t max_raw = 0, max_layer = 0;
    for (auto &ft : h.tensors) {
        auto it = lm->tensors.find(ft.name);
        JAS_CHECK(it != lm->tensors.end() && it->second.count != 0, JAS_ERR_INVALID,
                  "jas_lm_load: the file's tensor '" + ft.name + "' is not a weight of this model");
        const Tensor &t = it->second;
        const bool prefix_ok = ft.name == "wpe" && ft.rows >= t.rows;
        JAS_CHECK(ft.layers == t.layers && ft.cols == t.cols && (ft.rows == t.rows || prefix_ok), JAS_ERR_INVALID,
                  "jas_lm_load: '" + ft.name + "' has shape [" + std::to_string(ft.layers) + "," +
                      std::to_string(ft.rows) + "," + std::to_string(ft.cols) + "], the model needs [" +
                      std::to_string(t.layers) + "," + std::to_string(t.rows) + "," + std::to_string(t.cols) + "]");
        const size_t ne = (size_t)(t.packed ? 1 : t.layers) * t.rows * t.cols;  // one unit of upload
        max_raw = std::max(max_raw, ne * (ft.bf16 ? 2 : 4));
        if (t.packed || ft.bf16) max_layer = std::max(max_layer, ne);
    }
    for (auto &kv : lm->tensors)
        JAS_CHECK(kv.second.count == 0 || h.find(kv.first), JAS_ERR_INVALID,
                  "jas_lm_load: the file lacks '" + kv.first + "'");
    DevBuf raw, wide;
    if (max_raw) JAS_HIP(hipMalloc(&raw.p, max_raw));
    if (max_layer) JAS_HIP(hipMalloc(&wide.p, max_layer * sizeof(float)));
    Staging sg;
    TRY(sg.init());
    for (auto &ft : h.tensors) {
        const Tensor &t = lm->tensors.find(ft.name)->second;
        const std::string what = "jas_lm_load: " + ft.name;
        const size_t es = ft.bf16 ? 2 : 4;
        float *dev = lm->arena + t.off;
        const unsigned long long base = h.data_start + ft.begin;
        if (!t.packed) {
            const long ne = (long)t.layers * t.rows * t.cols;  // a prefix of wpe when longer
            if (!ft.bf16) {
                TRY(upload(f.fd, base, ne * es, dev, sg, s, what));
            } else {
                TRY(upload(f.fd, base, ne * es, raw.p, sg, s, what));
                hipLaunchKernelGGL(widen_bf16_kernel, dim3(ceil_div(ne, 256)), dim3(256), 0, s,
                                   (const uint16_t *)raw.p, dev, ne);
            }
            continue;
        }
        const long ne = (long)t.rows * t.cols;
        for (int l = 0; l < t.layers; ++l) {
            // the raw buffer is reused per layer: stream order keeps the pack of layer l
            // ahead of the copy of layer l + 1
            TRY(upload(f.fd, base + (unsigned long long)l * ne * es, ne * es, raw.p, sg, s, what));
            const float *src = (const float *)raw.p;
            if (ft.bf16) {
                hipLaunchKernelGGL(widen_bf16_kernel, dim3(ceil_div(ne, 256)), dim3(256), 0, s,
                                   (const uint16_t *)raw.p, (float *)wide.p, ne);
                src = (const float *)wide.p;
            }
            TRY(weight_pack(src, dev + l * t.lstride(), t.rows, t.cols, false, s, t.bf16));
        }
    }
    JAS_HIP(hipStreamSynchronize(s));
    return JAS_OK;
}

} // extern "C"
