// files.hip -- weight files into HBM: a bounded GGUF reader
// (components/cli/crates/spm-gguf/src/{parse,wire,tensor}.rs), the .spm
// forward-only reader and writer (components/format/crates/spm-file,
// spm-header, spm-layout, spm-walk; byte layout docs/spm-format.md), and the
// uploads that place their tensors in device memory.
//
// GGUF: the header, metadata and tensor directory are parsed under the
// reference's limits and with its error texts; tensor bodies are only reached
// through range reads bounded by a caller cap.  An upload streams a range from
// the file through two pinned host buffers, so the read of one chunk overlaps
// the DMA of the previous one, straight to its place in HBM.
//
// .spm: the reader walks (stream, group) forward exactly as spm_walk::Cursor
// does and hands out each group's scale and packed bytes.  A block-encoded
// stream (Q6K, Q5K, Q8_0: GGUF blocks in source row-major order, each scale
// group framed by a 4-byte inert f32 scale) goes to the device framed, in one
// copy, and a gather kernel drops the scales, leaving the blocks back to back
// as the matvec kernels read them.  An F32 stream (column-major: position k is
// W[k % rows][k / rows]) is gathered into row-major W.
#include "internal.hpp"

#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <new>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

namespace {

// spm-gguf/src/lib.rs:11-16
constexpr uint64_t kMaxMetadata = 1000000;
constexpr uint64_t kMaxTensors = 1000000;
constexpr uint64_t kMaxString = 16ull * 1024 * 1024;
constexpr uint64_t kMaxArray = 2000000;
constexpr uint32_t kMaxDims = 8;
constexpr uint64_t kMaxHeaderBytes = 512ull * 1024 * 1024;

constexpr size_t kStageBytes = 64ull << 20; // per pinned staging buffer

std::string fmt(const char *f, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// (elements, bytes) per block of a GGML dtype (spm-gguf/src/parse.rs:10-29).
bool ggml_layout(uint32_t t, uint64_t *block, uint64_t *size)
{
    switch (t) {
    case 0: *block = 1; *size = 4; return true;
    case 1: case 30: *block = 1; *size = 2; return true;
    case 2: *block = 32; *size = 18; return true;
    case 3: *block = 32; *size = 20; return true;
    case 6: *block = 32; *size = 22; return true;
    case 7: *block = 32; *size = 24; return true;
    case 8: *block = 32; *size = 34; return true;
    case 9: *block = 32; *size = 40; return true;
    case 10: *block = 256; *size = 84; return true;
    case 11: *block = 256; *size = 110; return true;
    case 12: *block = 256; *size = 144; return true;
    case 13: *block = 256; *size = 176; return true;
    case 14: *block = 256; *size = 210; return true;
    case 15: *block = 256; *size = 292; return true;
    case 16: *block = 1; *size = 8; return true;
    default: return false;
    }
}

// Strict UTF-8 (no overlong forms, no surrogates, nothing past U+10FFFF), the
// acceptance of String::from_utf8.
bool valid_utf8(const uint8_t *s, size_t n)
{
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) len = 2;
        else if (c == 0xe0) { len = 3; lo = 0xa0; }
        else if (c >= 0xe1 && c <= 0xec) len = 3;
        else if (c == 0xed) { len = 3; hi = 0x9f; }
        else if (c >= 0xee && c <= 0xef) len = 3;
        else if (c == 0xf0) { len = 4; lo = 0x90; }
        else if (c >= 0xf1 && c <= 0xf3) len = 4;
        else if (c == 0xf4) { len = 4; hi = 0x8f; }
        else return false;
        if (i + len > n) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (int k = 2; k < len; ++k)
            if (s[i + k] < 0x80 || s[i + k] > 0xbf) return false;
        i += len;
    }
    return true;
}

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t dtype = 0;
    uint64_t offset = 0; // absolute file offset
    uint64_t len = 0;
};

// Sequential reader over the header (spm-gguf/src/wire.rs:4-91).
struct Wire {
    int fd;
    uint64_t pos = 0, len = 0;
    std::vector<uint8_t> buf; // read-ahead window
    uint64_t buf_at = 0;      // file offset of buf[0]
    std::string err;

    bool bytes(uint64_t n, uint8_t *out)
    {
        uint64_t end;
        if (__builtin_add_overflow(pos, n, &end)) return fail("file position overflow");
        if (end > kMaxHeaderBytes) return fail("GGUF header exceeds limit");
        if (end > len) return fail("unexpected end of GGUF");
        uint64_t done = 0;
        while (done < n) {
            const uint64_t at = pos + done;
            if (at < buf_at || at >= buf_at + buf.size()) {
                const uint64_t want = std::min<uint64_t>(1ull << 20, len - at);
                buf.resize(want);
                uint64_t got = 0;
                while (got < want) {
                    const ssize_t r = pread(fd, buf.data() + got, want - got, (off_t)(at + got));
                    if (r < 0 && errno == EINTR) continue;
                    if (r <= 0) return fail(r < 0 ? strerror(errno) : "failed to fill whole buffer");
                    got += (uint64_t)r;
                }
                buf_at = at;
            }
            const uint64_t off = at - buf_at;
            const uint64_t take = std::min<uint64_t>(n - done, buf.size() - off);
            if (out) memcpy(out + done, buf.data() + off, take);
            done += take;
        }
        pos = end;
        return true;
    }
    bool fail(const std::string &m)
    {
        if (err.empty()) err = m;
        return false;
    }
    template <class T> bool scalar(T *v)
    {
        uint8_t b[sizeof(T)];
        if (!bytes(sizeof(T), b)) return false;
        memcpy(v, b, sizeof(T)); // little-endian host
        return true;
    }
    bool string(std::string *s)
    {
        uint64_t n;
        if (!scalar(&n)) return false;
        if (n > kMaxString) return fail(fmt("string length %llu exceeds limit", (unsigned long long)n));
        std::string v(n, '\0');
        if (!bytes(n, reinterpret_cast<uint8_t *>(v.data()))) return false;
        if (!valid_utf8(reinterpret_cast<const uint8_t *>(v.data()), n)) return fail("invalid UTF-8 string");
        *s = std::move(v);
        return true;
    }
    // One metadata value; scalars and strings render as the reference's
    // to_string() does, the others (f32, f64, arrays) as "<type>".  The numeric
    // value of a scalar, floats included, is kept beside the rendering.
    bool value(uint32_t ty, int depth, std::string *out, double *num, bool *has_num)
    {
        if (depth > 4) return fail("metadata nesting exceeds limit");
        *has_num = false;
        char b[32];
        switch (ty) {
        case 0: { uint8_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%u", v); *num = v; break; }
        case 1: { int8_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%d", v); *num = v; break; }
        case 2: { uint16_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%u", v); *num = v; break; }
        case 3: { int16_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%d", v); *num = v; break; }
        case 4: { uint32_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%u", v); *num = v; break; }
        case 5: { int32_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%d", v); *num = v; break; }
        case 6: {
            float v;
            if (!scalar(&v)) return false;
            *out = "<6>";
            *num = v;
            *has_num = true;
            return true;
        }
        case 7: {
            uint8_t v;
            if (!scalar(&v)) return false;
            if (v > 1) return fail("invalid boolean metadata value");
            snprintf(b, sizeof b, "%u", v);
            *num = v;
            break;
        }
        case 8: return string(out);
        case 9: {
            uint32_t inner;
            uint64_t n;
            if (!scalar(&inner) || !scalar(&n)) return false;
            if (n > kMaxArray) return fail(fmt("array length %llu exceeds limit", (unsigned long long)n));
            std::string sink;
            double d;
            bool h;
            for (uint64_t i = 0; i < n; ++i)
                if (!value(inner, depth + 1, &sink, &d, &h)) return false;
            *out = "<9>";
            return true;
        }
        case 10: { uint64_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%llu", (unsigned long long)v); *num = (double)v; break; }
        case 11: { int64_t v; if (!scalar(&v)) return false; snprintf(b, sizeof b, "%lld", (long long)v); *num = (double)v; break; }
        case 12: {
            double v;
            if (!scalar(&v)) return false;
            *out = "<12>";
            *num = v;
            *has_num = true;
            return true;
        }
        default: return fail(fmt("unknown metadata type %u", ty));
        }
        *out = b;
        *has_num = true;
        return true;
    }
};

} // namespace

struct emu_gguf {
    int fd = -1;
    uint64_t file_len = 0;
    uint32_t version = 0;
    uint64_t metadata_count = 0;
    uint64_t data_offset = 0;
    std::vector<std::string> keys, values; // file order
    std::vector<double> numbers;
    std::vector<uint8_t> has_number;
    std::vector<GgufTensor> tensors; // ascending offset
    std::string error;

    int failed(int status, const std::string &m)
    {
        error = m;
        return status;
    }
};

namespace {

// spm-gguf/src/parse.rs:157-182 (read), with prelude :31-48, metadata :50-63,
// descriptors :65-92, ranges :94-140 and reject_overlaps :142-154.
int gguf_parse(emu_gguf *g)
{
    Wire p;
    p.fd = g->fd;
    p.len = g->file_len;
    uint8_t magic[4];
    if (!p.bytes(4, magic)) return g->failed(EMU_E_FORMAT, p.err);
    if (memcmp(magic, "GGUF", 4) != 0) return g->failed(EMU_E_FORMAT, "invalid GGUF magic");
    uint32_t version;
    uint64_t tensors, metadata;
    if (!p.scalar(&version)) return g->failed(EMU_E_FORMAT, p.err);
    if (version != 3) return g->failed(EMU_E_FORMAT, fmt("unsupported GGUF version %u", version));
    if (!p.scalar(&tensors) || !p.scalar(&metadata)) return g->failed(EMU_E_FORMAT, p.err);
    if (tensors > kMaxTensors) return g->failed(EMU_E_FORMAT, "tensor count exceeds limit");
    if (metadata > kMaxMetadata) return g->failed(EMU_E_FORMAT, "metadata count exceeds limit");
    g->version = version;
    g->metadata_count = metadata;
    std::unordered_set<std::string> seen;
    for (uint64_t i = 0; i < metadata; ++i) {
        std::string key, val;
        uint32_t ty;
        double num = 0;
        bool has = false;
        if (!p.string(&key) || !p.scalar(&ty) || !p.value(ty, 0, &val, &num, &has))
            return g->failed(EMU_E_FORMAT, p.err);
        if (!seen.insert(key).second) return g->failed(EMU_E_FORMAT, "duplicate metadata key");
        g->keys.push_back(std::move(key));
        g->values.push_back(std::move(val));
        g->numbers.push_back(num);
        g->has_number.push_back(has ? 1 : 0);
    }
    std::vector<GgufTensor> raw;
    std::unordered_set<std::string> names;
    for (uint64_t i = 0; i < tensors; ++i) {
        GgufTensor t;
        if (!p.string(&t.name)) return g->failed(EMU_E_FORMAT, p.err);
        if (!names.insert(t.name).second) return g->failed(EMU_E_FORMAT, "duplicate tensor name " + t.name);
        uint32_t nd;
        if (!p.scalar(&nd)) return g->failed(EMU_E_FORMAT, p.err);
        if (nd == 0 || nd > kMaxDims) return g->failed(EMU_E_FORMAT, fmt("invalid dimension count %u", nd));
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            if (!p.scalar(&t.dims[d])) return g->failed(EMU_E_FORMAT, p.err);
        if (!p.scalar(&t.dtype) || !p.scalar(&t.offset)) return g->failed(EMU_E_FORMAT, p.err);
        raw.push_back(std::move(t));
    }
    uint64_t align = 32;
    for (size_t i = 0; i < g->keys.size(); ++i) {
        if (g->keys[i] != "general.alignment") continue;
        // "parse::<u64>()": an optional '+' then decimal digits that fit
        // u64; anything else keeps 32
        const std::string &v = g->values[i];
        const size_t k0 = (!v.empty() && v[0] == '+') ? 1 : 0;
        bool ok = v.size() > k0;
        unsigned long long x = 0;
        for (size_t k = k0; k < v.size(); ++k) {
            const char c = v[k];
            if (c < '0' || c > '9') { ok = false; break; }
            if (__builtin_mul_overflow(x, 10ull, &x) || __builtin_add_overflow(x, (unsigned long long)(c - '0'), &x)) {
                ok = false;
                break;
            }
        }
        if (ok) align = x;
    }
    if (align == 0 || (align & (align - 1)) != 0) return g->failed(EMU_E_FORMAT, "invalid alignment");
    uint64_t base;
    if (__builtin_add_overflow(p.pos, align - 1, &base)) return g->failed(EMU_E_FORMAT, "alignment overflow");
    base &= ~(align - 1);
    if (base > g->file_len) return g->failed(EMU_E_FORMAT, "tensor data starts beyond file");
    g->data_offset = base;
    for (GgufTensor &r : raw) {
        if (r.offset % align != 0) return g->failed(EMU_E_FORMAT, "unaligned tensor " + r.name);
        for (uint64_t d : r.dims)
            if (d == 0) return g->failed(EMU_E_FORMAT, "tensor " + r.name + " has a zero dimension");
        uint64_t elems = 1;
        for (uint64_t d : r.dims)
            if (__builtin_mul_overflow(elems, d, &elems))
                return g->failed(EMU_E_FORMAT, "tensor element count overflow");
        uint64_t block, size;
        if (!ggml_layout(r.dtype, &block, &size))
            return g->failed(EMU_E_FORMAT, fmt("unsupported GGML dtype %u", r.dtype));
        if (elems % block != 0) return g->failed(EMU_E_FORMAT, "tensor " + r.name + " does not fill dtype blocks");
        uint64_t len, off, end;
        if (__builtin_mul_overflow(elems / block, size, &len))
            return g->failed(EMU_E_FORMAT, "tensor byte length overflow");
        if (__builtin_add_overflow(base, r.offset, &off)) return g->failed(EMU_E_FORMAT, "tensor offset overflow");
        if (__builtin_add_overflow(off, len, &end)) return g->failed(EMU_E_FORMAT, "tensor end overflow");
        if (end > g->file_len) return g->failed(EMU_E_FORMAT, "tensor " + r.name + " extends beyond file");
        r.offset = off;
        r.len = len;
    }
    std::stable_sort(raw.begin(), raw.end(),
                     [](const GgufTensor &a, const GgufTensor &b) { return a.offset < b.offset; });
    for (size_t i = 1; i < raw.size(); ++i)
        if (raw[i - 1].offset + raw[i - 1].len > raw[i].offset)
            return g->failed(EMU_E_FORMAT, "overlapping tensor ranges");
    g->tensors = std::move(raw);
    return EMU_OK;
}

// spm-gguf/src/tensor.rs:35-67 (read_tensor_range): the checks, in order.
int gguf_check_range(emu_gguf *g, uint64_t index, uint64_t rel, uint64_t len, uint64_t max_bytes,
                     uint64_t *abs_off)
{
    if (index >= g->tensors.size()) return g->failed(EMU_E_ARG, "tensor index out of range");
    const GgufTensor &t = g->tensors[index];
    if (len > max_bytes)
        return g->failed(EMU_E_ARG, fmt("tensor %s request is %llu bytes, exceeding limit %llu", t.name.c_str(),
                                        (unsigned long long)len, (unsigned long long)max_bytes));
    uint64_t rend;
    if (__builtin_add_overflow(rel, len, &rend)) return g->failed(EMU_E_ARG, "tensor range overflow");
    if (rend > t.len) return g->failed(EMU_E_ARG, "requested range exceeds tensor " + t.name);
    if (__builtin_add_overflow(t.offset, rel, abs_off)) return g->failed(EMU_E_ARG, "tensor offset overflow");
    return EMU_OK;
}

int read_exact(emu_gguf *g, uint64_t off, void *dst, uint64_t n)
{
    uint8_t *d = static_cast<uint8_t *>(dst);
    uint64_t got = 0;
    while (got < n) {
        const size_t want = (size_t)std::min<uint64_t>(n - got, 1ull << 30);
        const ssize_t r = pread(g->fd, d + got, want, (off_t)(off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) return g->failed(EMU_E_IO, strerror(errno));
        if (r == 0) return g->failed(EMU_E_IO, "failed to fill whole buffer");
        got += (uint64_t)r;
    }
    return EMU_OK;
}

int ensure_stage(emu_ctx *ctx)
{
    if (ctx->stage_bytes) return EMU_OK;
    for (int i = 0; i < 2; ++i) {
        EMU_HIP(ctx, hipHostMalloc(&ctx->stage[i], kStageBytes, hipHostMallocDefault));
        EMU_HIP(ctx, hipEventCreateWithFlags(&ctx->stage_ev[i], hipEventDisableTiming));
    }
    ctx->stage_bytes = kStageBytes;
    return EMU_OK;
}

// ------------------------------------------------------------- .spm -------

// spm-layout/src/model.rs:80-91 (Encoding::bytes_for), codes :111-121.
bool spm_bytes_for(uint32_t enc, uint64_t count, uint64_t *bytes)
{
    switch (enc) {
    case EMU_SPM_TERNARY: *bytes = (count + 3) / 4; return true;
    case EMU_SPM_F32: *bytes = count * 4; return true;
    case EMU_SPM_BF16: *bytes = count * 2; return true;
    case EMU_SPM_Q6K: *bytes = (count + 255) / 256 * 210; return true;
    case EMU_SPM_Q5K: *bytes = (count + 255) / 256 * 176; return true;
    case EMU_SPM_Q8_0: *bytes = (count + 31) / 32 * 34; return true;
    default: return false;
    }
}

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
void wr32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }

constexpr uint8_t kSpmMagic[8] = {0x89, 'S', 'P', 'M', 0x0D, 0x0A, 0x1A, 0x0A};
constexpr size_t kSpmHeader = 32, kSpmDescriptor = 32, kSpmScale = 4;
constexpr uint16_t kSpmMajor = 1, kSpmMinor = 0;

// Forward position in the (stream, group) sequence (spm-walk/src/cursor.rs:6-58,
// spm-layout/src/tiling.rs:4-51).
struct SpmCursor {
    uint32_t stream = 0;
    uint64_t group = 0;

    static uint64_t total(const emu_spm_descriptor &d) { return (uint64_t)d.rows * d.cols; }
    static uint64_t groups(const emu_spm_descriptor &d) { return (total(d) + d.group_size - 1) / d.group_size; }
    void settle(const std::vector<emu_spm_descriptor> &ds)
    {
        while (stream < ds.size()) {
            if (group < groups(ds[stream])) return;
            ++stream;
            group = 0;
        }
    }
    bool group_len(const std::vector<emu_spm_descriptor> &ds, uint32_t *len) const
    {
        if (stream >= ds.size()) return false;
        const emu_spm_descriptor &d = ds[stream];
        const uint64_t t = total(d), start = (uint64_t)d.group_size * group;
        *len = start >= t ? 0 : (uint32_t)std::min<uint64_t>(t - start, d.group_size);
        return true;
    }
    void advance(const std::vector<emu_spm_descriptor> &ds)
    {
        if (stream >= ds.size()) return;
        ++group;
        settle(ds);
    }
};

// spm-layout/src/wire.rs:12-29 (parse): length, then group_size, then encoding.
int spm_parse_descriptor(const uint8_t *src, size_t avail, emu_spm_descriptor *d, std::string *err)
{
    if (avail < kSpmDescriptor) {
        *err = fmt("descriptor truncated: %zu bytes, need 32", avail);
        return EMU_E_FORMAT;
    }
    const uint32_t gs = rd32(src + 8);
    if (gs == 0) {
        *err = "group_size must be at least 1";
        return EMU_E_FORMAT;
    }
    uint64_t probe;
    if (!spm_bytes_for(src[12], 1, &probe)) {
        *err = fmt("unknown .spm encoding profile %u", src[12]);
        return EMU_E_FORMAT;
    }
    d->rows = rd32(src);
    d->cols = rd32(src + 4);
    d->group_size = gs;
    d->encoding = src[12];
    d->lane_count = rd16(src + 14);
    return EMU_OK;
}

// Drop each group's 4-byte scale: out[g*P + i] = framed[g*(P+4) + 4 + i].
// P is even for every block encoding, so the copy moves 16-bit halves.
__global__ __launch_bounds__(256) void spm_unframe_kernel(const uint8_t *framed, uint8_t *out, uint64_t halves,
                                                          uint32_t p_halves)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= halves) return;
    const uint64_t g = i / p_halves, w = i - g * p_halves;
    const uint64_t src = g * (2ull * p_halves + kSpmScale) + kSpmScale + 2 * w;
    uint16_t v;
    __builtin_memcpy(&v, framed + src, 2);
    __builtin_memcpy(out + 2 * i, &v, 2);
}

// F32 stream, column-major with scale groups of gs weights, into row-major
// rows x cols: out[r*cols + c] = weight at position k = c*rows + r.
__global__ __launch_bounds__(256) void spm_f32_rows_kernel(const uint8_t *framed, float *out, uint32_t rows,
                                                           uint32_t cols, uint32_t gs)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t n = (uint64_t)rows * cols;
    if (i >= n) return;
    const uint64_t r = i / cols, c = i - r * cols;
    const uint64_t k = c * rows + r, g = k / gs, w = k - g * gs;
    const uint64_t src = g * (kSpmScale + 4ull * gs) + kSpmScale + 4 * w;
    float v;
    __builtin_memcpy(&v, framed + src, 4);
    out[i] = v;
}

} // namespace

struct emu_spm {
    const uint8_t *src = nullptr; // borrowed: the caller keeps the bytes alive
    size_t len = 0;
    uint16_t major = 0, minor = 0;
    uint32_t stream_count = 0;
    std::vector<emu_spm_descriptor> desc;
    size_t payload = 0; // offset of the payload in src
    size_t at = 0;      // bytes of payload consumed
    SpmCursor cur;
    std::string error;
};

struct emu_spm_writer {
    std::vector<emu_spm_descriptor> desc;
    std::vector<uint8_t> out;
    SpmCursor cur;
    std::string error;
};

// ============================================================== C ABI ====

extern "C" int emu_gguf_open(const char *path, emu_gguf **out, char *h_err, size_t err_len)
{
    if (h_err && err_len) h_err[0] = '\0';
    if (!path || !out) return EMU_E_ARG;
    *out = nullptr;
    emu_gguf *g = new (std::nothrow) emu_gguf();
    if (!g) return EMU_E_NOMEM;
    int st = EMU_OK;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat sb;
    if (g->fd < 0) st = g->failed(EMU_E_IO, fmt("%s: %s", path, strerror(errno)));
    else if (fstat(g->fd, &sb) != 0) st = g->failed(EMU_E_IO, strerror(errno));
    else {
        g->file_len = (uint64_t)sb.st_size;
        try {
            st = gguf_parse(g);
        } catch (const std::bad_alloc &) {
            st = g->failed(EMU_E_NOMEM, "allocation refused");
        }
    }
    if (st != EMU_OK) {
        if (h_err && err_len) snprintf(h_err, err_len, "%s", g->error.c_str());
        if (g->fd >= 0) close(g->fd);
        delete g;
        return st;
    }
    *out = g;
    return EMU_OK;
}

extern "C" int emu_gguf_close(emu_gguf *g)
{
    if (!g) return EMU_E_ARG;
    if (g->fd >= 0) close(g->fd);
    delete g;
    return EMU_OK;
}

extern "C" const char *emu_gguf_error(const emu_gguf *g) { return g ? g->error.c_str() : ""; }

extern "C" int emu_gguf_summary(const emu_gguf *g, uint32_t *version, uint64_t *metadata_count,
                                uint64_t *tensor_data_offset, uint64_t *tensor_count)
{
    if (!g) return EMU_E_ARG;
    if (version) *version = g->version;
    if (metadata_count) *metadata_count = g->metadata_count;
    if (tensor_data_offset) *tensor_data_offset = g->data_offset;
    if (tensor_count) *tensor_count = g->tensors.size();
    return EMU_OK;
}

extern "C" int emu_gguf_metadata_at(const emu_gguf *g, uint64_t index, const char **key, size_t *key_len,
                                    const char **value, size_t *value_len)
{
    if (!g || !key || !value || index >= g->keys.size()) return EMU_E_ARG;
    *key = g->keys[index].c_str();
    *value = g->values[index].c_str();
    if (key_len) *key_len = g->keys[index].size();
    if (value_len) *value_len = g->values[index].size();
    return EMU_OK;
}

extern "C" int emu_gguf_metadata_number(const emu_gguf *g, const char *key, double *value)
{
    if (!g || !key || !value) return EMU_E_ARG;
    for (size_t i = 0; i < g->keys.size(); ++i)
        if (g->keys[i] == key) {
            if (!g->has_number[i]) return EMU_E_UNSUPPORTED;
            *value = g->numbers[i];
            return EMU_OK;
        }
    return EMU_E_ARG;
}

extern "C" int emu_gguf_tensor_at(const emu_gguf *g, uint64_t index, emu_gguf_tensor_info *info)
{
    if (!g || !info || index >= g->tensors.size()) return EMU_E_ARG;
    const GgufTensor &t = g->tensors[index];
    info->name = t.name.c_str();
    info->name_len = t.name.size();
    info->n_dims = (uint32_t)t.dims.size();
    for (uint32_t d = 0; d < 8; ++d) info->dims[d] = d < t.dims.size() ? t.dims[d] : 0;
    info->dtype = t.dtype;
    info->offset = t.offset;
    info->len = t.len;
    return EMU_OK;
}

extern "C" int emu_gguf_find(emu_gguf *g, const char *name, uint64_t *index)
{
    if (!g || !name || !index) return EMU_E_ARG;
    for (size_t i = 0; i < g->tensors.size(); ++i)
        if (g->tensors[i].name == name) {
            *index = i;
            return EMU_OK;
        }
    return g->failed(EMU_E_FORMAT, std::string("missing tensor ") + name);
}

extern "C" int emu_gguf_read_range(emu_gguf *g, uint64_t index, uint64_t rel_off, uint64_t len,
                                   uint64_t max_bytes, void *h_dst)
{
    if (!g || (!h_dst && len)) return EMU_E_ARG;
    uint64_t off;
    int st = gguf_check_range(g, index, rel_off, len, max_bytes, &off);
    if (st != EMU_OK) return st;
    return read_exact(g, off, h_dst, len);
}

extern "C" int emu_gguf_upload(emu_ctx *ctx, emu_gguf *g, uint64_t index, uint64_t rel_off, uint64_t len,
                               void *d_dst)
{
    if (!ctx || !g || (!d_dst && len)) return EMU_E_ARG;
    uint64_t off;
    int st = gguf_check_range(g, index, rel_off, len, len, &off);
    if (st != EMU_OK) return st;
    if ((st = ensure_stage(ctx)) != EMU_OK) return st;
    uint8_t *dst = static_cast<uint8_t *>(d_dst);
    int k = 0;
    for (uint64_t done = 0; done < len; done += ctx->stage_bytes, k ^= 1) {
        const uint64_t n = std::min<uint64_t>(len - done, ctx->stage_bytes);
        // The buffer's previous copy must have left before it is refilled.
        EMU_HIP(ctx, hipEventSynchronize(ctx->stage_ev[k]));
        if ((st = read_exact(g, off + done, ctx->stage[k], n)) != EMU_OK) {
            (void)hipStreamSynchronize(ctx->stream);
            return st;
        }
        EMU_HIP(ctx, hipMemcpyAsync(dst + done, ctx->stage[k], n, hipMemcpyHostToDevice, ctx->stream));
        EMU_HIP(ctx, hipEventRecord(ctx->stage_ev[k], ctx->stream));
    }
    EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return EMU_OK;
}

extern "C" int emu_spm_bytes_for(uint32_t encoding, uint64_t count, uint64_t *bytes)
{
    if (!bytes) return EMU_E_ARG;
    return spm_bytes_for(encoding, count, bytes) ? EMU_OK : EMU_E_UNSUPPORTED;
}

extern "C" int emu_spm_parse(const void *h_bytes, size_t len, emu_spm **out, char *h_err, size_t err_len)
{
    if (h_err && err_len) h_err[0] = '\0';
    if (!out || (!h_bytes && len)) return EMU_E_ARG;
    *out = nullptr;
    const uint8_t *src = static_cast<const uint8_t *>(h_bytes);
    std::string err;
    int st = EMU_OK;
    // spm-header/src/parse.rs:12-58
    if (len < kSpmHeader) {
        err = fmt("header truncated: %zu bytes available, need 32", len);
        st = EMU_E_FORMAT;
    } else if (memcmp(src, kSpmMagic, 8) != 0) {
        err = "bad magic: not a .spm file, or corrupted in transit";
        st = EMU_E_FORMAT;
    } else if (rd16(src + 8) > kSpmMajor) {
        err = fmt("unsupported .spm major version %u: this build reads up to %u", rd16(src + 8), kSpmMajor);
        st = EMU_E_FORMAT;
    } else if (src[12] != 0) {
        err = fmt("unknown endianness discriminant %u", src[12]);
        st = EMU_E_FORMAT;
    }
    if (st != EMU_OK) {
        if (h_err && err_len) snprintf(h_err, err_len, "%s", err.c_str());
        return st;
    }
    emu_spm *r = new (std::nothrow) emu_spm();
    if (!r) return EMU_E_NOMEM;
    r->src = src;
    r->len = len;
    r->major = rd16(src + 8);
    r->minor = rd16(src + 10);
    r->stream_count = rd32(src + 16);
    // spm-file/src/read.rs:48-63: one descriptor after another; a file that
    // ends inside the directory fails on the first short descriptor.
    size_t at = kSpmHeader;
    try {
        for (uint32_t i = 0; i < r->stream_count; ++i) {
            emu_spm_descriptor d{};
            const size_t avail = at <= len ? len - at : 0;
            if ((st = spm_parse_descriptor(src + std::min(at, len), avail, &d, &err)) != EMU_OK) break;
            r->desc.push_back(d);
            at += kSpmDescriptor;
        }
    } catch (const std::bad_alloc &) {
        st = EMU_E_NOMEM;
        err = "allocation refused";
    }
    if (st != EMU_OK) {
        if (h_err && err_len) snprintf(h_err, err_len, "%s", err.c_str());
        delete r;
        return st;
    }
    r->payload = std::min(at, len);
    r->cur.settle(r->desc);
    *out = r;
    return EMU_OK;
}

extern "C" int emu_spm_close(emu_spm *r)
{
    if (!r) return EMU_E_ARG;
    delete r;
    return EMU_OK;
}

extern "C" const char *emu_spm_error(const emu_spm *r) { return r ? r->error.c_str() : ""; }

extern "C" int emu_spm_header(const emu_spm *r, uint16_t *major, uint16_t *minor, uint32_t *stream_count)
{
    if (!r) return EMU_E_ARG;
    if (major) *major = r->major;
    if (minor) *minor = r->minor;
    if (stream_count) *stream_count = r->stream_count;
    return EMU_OK;
}

extern "C" int emu_spm_descriptor_at(const emu_spm *r, uint32_t index, emu_spm_descriptor *d)
{
    if (!r || !d || index >= r->desc.size()) return EMU_E_ARG;
    *d = r->desc[index];
    return EMU_OK;
}

extern "C" int emu_spm_position(const emu_spm *r, uint32_t *stream, uint64_t *group)
{
    if (!r) return EMU_E_ARG;
    if (stream) *stream = r->cur.stream;
    if (group) *group = r->cur.group;
    return EMU_OK;
}

extern "C" int emu_spm_next_group(emu_spm *r, int *has_group, emu_spm_group *grp)
{
    if (!r || !has_group || !grp) return EMU_E_ARG;
    uint32_t count;
    if (!r->cur.group_len(r->desc, &count)) {
        *has_group = 0;
        return EMU_OK;
    }
    *has_group = 1;
    uint64_t bytes;
    spm_bytes_for(r->desc[r->cur.stream].encoding, count, &bytes);
    const size_t plen = r->len - r->payload;
    const uint64_t needed = kSpmScale + bytes;
    const uint64_t available = plen > r->at ? plen - r->at : 0;
    if (needed > available) {
        r->error = fmt("payload truncated: group needs %llu bytes, %llu remain", (unsigned long long)needed,
                       (unsigned long long)available);
        return EMU_E_TRUNCATED;
    }
    const uint8_t *g = r->src + r->payload + r->at;
    grp->stream = r->cur.stream;
    uint32_t sbits = rd32(g);
    memcpy(&grp->scale, &sbits, 4);
    grp->count = count;
    grp->packed = g + kSpmScale;
    grp->packed_len = (size_t)bytes;
    r->at += (size_t)needed;
    r->cur.advance(r->desc);
    return EMU_OK;
}

extern "C" int emu_spm_upload_stream(emu_ctx *ctx, emu_spm *r, void *d_dst, size_t dst_len, uint32_t *stream)
{
    if (!ctx || !r || !d_dst) return EMU_E_ARG;
    if (r->cur.stream >= r->desc.size()) {
        r->error = "no stream left to read";
        return EMU_E_ARG;
    }
    if (r->cur.group != 0) {
        r->error = fmt("reader is inside stream %u (group %llu), not at its start", r->cur.stream,
                       (unsigned long long)r->cur.group);
        return EMU_E_ARG;
    }
    const uint32_t s = r->cur.stream;
    const emu_spm_descriptor d = r->desc[s];
    if (d.encoding != EMU_SPM_Q6K && d.encoding != EMU_SPM_Q5K && d.encoding != EMU_SPM_Q8_0 &&
        d.encoding != EMU_SPM_F32) {
        r->error = fmt("stream %u: no device layout for encoding profile %u", s, d.encoding);
        return EMU_E_UNSUPPORTED;
    }
    const uint64_t total = (uint64_t)d.rows * d.cols;
    uint64_t be = 0, bb = 0; // block elements / bytes
    switch (d.encoding) {
    case EMU_SPM_Q6K: be = 256; bb = 210; break;
    case EMU_SPM_Q5K: be = 256; bb = 176; break;
    case EMU_SPM_Q8_0: be = 32; bb = 34; break;
    default: be = 1; bb = 4; break;
    }
    // Block streams: every group must hold whole blocks (a short block would
    // pad the matrix); F32: groups of any size.
    if (d.encoding != EMU_SPM_F32 && (d.group_size % be != 0 || total % be != 0)) {
        r->error = fmt("stream %u: group_size %u or %llu weights is not whole %llu-weight blocks", s, d.group_size,
                       (unsigned long long)total, (unsigned long long)be);
        return EMU_E_FORMAT;
    }
    const uint64_t out_bytes = total / be * bb;
    if (dst_len < out_bytes) {
        r->error = fmt("stream %u needs %llu device bytes, %zu given", s, (unsigned long long)out_bytes, dst_len);
        return EMU_E_ARG;
    }
    // Walk the stream's groups as next_group would, without consuming on failure.
    const size_t plen = r->len - r->payload;
    uint64_t framed = 0;
    for (uint64_t gi = 0;; ++gi) {
        const uint64_t start = gi * d.group_size;
        if (start >= total) break;
        const uint64_t count = std::min<uint64_t>(total - start, d.group_size);
        uint64_t bytes;
        spm_bytes_for(d.encoding, count, &bytes);
        const uint64_t avail = plen > r->at + framed ? plen - r->at - framed : 0;
        if (kSpmScale + bytes > avail) {
            r->error = fmt("payload truncated: group needs %llu bytes, %llu remain",
                           (unsigned long long)(kSpmScale + bytes), (unsigned long long)avail);
            return EMU_E_TRUNCATED;
        }
        framed += kSpmScale + bytes;
    }
    const uint64_t threads = d.encoding == EMU_SPM_F32 ? total : out_bytes / 2;
    if ((threads + 255) / 256 > 0x7fffffffull) {
        r->error = fmt("stream %u is too large for one placement launch", s);
        return EMU_E_UNSUPPORTED;
    }
    const uint8_t *src = r->src + r->payload + r->at;
    void *tmp = nullptr;
    int st = emu_malloc(ctx, framed, &tmp);
    if (st != EMU_OK) return st;
    hipError_t e = hipMemcpyAsync(tmp, src, framed, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        if (d.encoding == EMU_SPM_F32) {
            const uint64_t n = total;
            hipLaunchKernelGGL(spm_f32_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream,
                               static_cast<const uint8_t *>(tmp), static_cast<float *>(d_dst), d.rows, d.cols,
                               d.group_size);
        } else {
            const uint64_t p_halves = d.group_size / be * bb / 2, halves = out_bytes / 2;
            hipLaunchKernelGGL(spm_unframe_kernel, dim3((unsigned)((halves + 255) / 256)), dim3(256), 0, ctx->stream,
                               static_cast<const uint8_t *>(tmp), static_cast<uint8_t *>(d_dst), halves,
                               (uint32_t)p_halves);
        }
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    emu_free(ctx, tmp);
    if (e != hipSuccess) return emu_hip_fail(ctx, e, "emu_spm_upload_stream");
    // Consume the stream: the cursor moves to the next stream's first group.
    r->at += (size_t)framed;
    r->cur.stream = s + 1;
    r->cur.group = 0;
    r->cur.settle(r->desc);
    if (stream) *stream = s;
    return EMU_OK;
}

extern "C" int emu_spm_writer_create(const emu_spm_descriptor *descs, uint32_t n, emu_spm_writer **out)
{
    if (!out || (!descs && n)) return EMU_E_ARG;
    *out = nullptr;
    emu_spm_writer *w = new (std::nothrow) emu_spm_writer();
    if (!w) return EMU_E_NOMEM;
    try {
        w->desc.assign(descs, descs + n);
        // spm-file/src/write.rs:23-36: header and directory up front.
        w->out.resize(kSpmHeader + (size_t)kSpmDescriptor * n, 0);
        uint8_t *h = w->out.data();
        memcpy(h, kSpmMagic, 8);
        wr16(h + 8, kSpmMajor);
        wr16(h + 10, kSpmMinor);
        h[12] = 0;
        wr32(h + 16, n);
        for (uint32_t i = 0; i < n; ++i) {
            uint8_t *p = h + kSpmHeader + (size_t)kSpmDescriptor * i;
            wr32(p, descs[i].rows);
            wr32(p + 4, descs[i].cols);
            wr32(p + 8, descs[i].group_size);
            p[12] = (uint8_t)descs[i].encoding;
            wr16(p + 14, (uint16_t)descs[i].lane_count);
        }
    } catch (const std::bad_alloc &) {
        delete w;
        return EMU_E_NOMEM;
    }
    w->cur.settle(w->desc);
    *out = w;
    return EMU_OK;
}

extern "C" int emu_spm_write_raw_group(emu_spm_writer *w, float scale, const void *h_payload, size_t payload_len,
                                       uint64_t count)
{
    if (!w || (!h_payload && payload_len)) return EMU_E_ARG;
    uint32_t expected;
    if (!w->cur.group_len(w->desc, &expected)) {
        w->error = fmt("only %u of %zu streams were written", w->cur.stream, w->desc.size());
        return EMU_E_FORMAT;
    }
    uint64_t bytes = 0;
    const bool known = spm_bytes_for(w->desc[w->cur.stream].encoding, count, &bytes);
    if (count != expected || !known || payload_len != bytes) {
        w->error = fmt("group expects %u weights, got %llu", expected, (unsigned long long)count);
        return EMU_E_SHAPE;
    }
    try {
        uint8_t sb[4];
        uint32_t bits;
        memcpy(&bits, &scale, 4);
        wr32(sb, bits);
        w->out.insert(w->out.end(), sb, sb + 4);
        const uint8_t *p = static_cast<const uint8_t *>(h_payload);
        w->out.insert(w->out.end(), p, p + payload_len);
    } catch (const std::bad_alloc &) {
        return EMU_E_NOMEM;
    }
    w->cur.advance(w->desc);
    return EMU_OK;
}

extern "C" int emu_spm_writer_finish(emu_spm_writer *w, const uint8_t **h_bytes, size_t *len)
{
    if (!w || !h_bytes || !len) return EMU_E_ARG;
    if (w->cur.stream != w->desc.size()) {
        w->error = fmt("only %u of %zu streams were written", w->cur.stream, w->desc.size());
        return EMU_E_FORMAT;
    }
    *h_bytes = w->out.data();
    *len = w->out.size();
    return EMU_OK;
}

extern "C" const char *emu_spm_writer_error(const emu_spm_writer *w) { return w ? w->error.c_str() : ""; }

extern "C" int emu_spm_writer_destroy(emu_spm_writer *w)
{
    if (!w) return EMU_E_ARG;
    delete w;
    return EMU_OK;
}
