// gguf.cpp -- bounds-checked GGUF v2/v3 reader (host only: no HIP call).
//
// Parses the whole header once at open, validating every record against the
// file size, and keeps per-key and per-tensor offsets so that later lookups
// are O(1) and never re-read the header.  The reference's reader
// (src/model/gguf.rs) walks the same records; the differences are listed in
// include/rrr_gguf.h.
#include "rrr_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "GGUF fields are read as host little-endian integers");

namespace rrr {
// Defined beside rrr_last_error(): stores the thread-local message (RRR_OK clears it).
int set_error(int code, const char *msg);
}  // namespace rrr

struct rrr_gguf {
    struct Kv {
        std::string key;
        uint32_t type, elem_type;
        uint64_t count;                // array elements / string bytes / 1
        uint64_t off, bytes;           // the value's payload in the file
        std::vector<uint64_t> strs;    // string arrays: offset of each element's u64 length
    };
    struct Tensor {
        std::string name;
        uint32_t n_dims, type;
        uint64_t dims[4];
        uint64_t offset, n_elements, bytes;
    };
    uint32_t magic;
    const uint8_t *base;
    uint64_t size;
    bool mapped;
    uint32_t version;
    uint64_t alignment, data_offset;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint64_t> kv_index, tensor_index;
};

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint32_t HANDLE_MAGIC = 0x52524746u;
constexpr int MAX_ARRAY_DEPTH = 4;            // arrays of arrays nest at most this deep
constexpr uint64_t MAX_ALIGNMENT = 1ull << 30;

std::mutex g_mu;
std::unordered_set<const rrr_gguf *> g_live;

int err(int code, const char *fmt, ...)
{
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    return rrr::set_error(code, msg);
}

int ok() { return rrr::set_error(RRR_OK, ""); }

using ull = unsigned long long;

// ggml's tensor types (enum ggml_type and its type traits): a block of
// `elems` elements is stored in `bytes` bytes.  Retired numbers (4, 5, 31-33,
// 36-38) are absent.
struct TypeSize {
    uint32_t elems, bytes;
    const char *name;
};
constexpr uint32_t N_TYPES = 40;
const TypeSize TYPES[N_TYPES] = {
    {1, 4, "F32"},      {1, 2, "F16"},       {32, 18, "Q4_0"},    {32, 20, "Q4_1"},   {0, 0, nullptr},
    {0, 0, nullptr},    {32, 22, "Q5_0"},    {32, 24, "Q5_1"},    {32, 34, "Q8_0"},   {32, 36, "Q8_1"},
    {256, 84, "Q2_K"},  {256, 110, "Q3_K"},  {256, 144, "Q4_K"},  {256, 176, "Q5_K"}, {256, 210, "Q6_K"},
    {256, 292, "Q8_K"}, {256, 66, "IQ2_XXS"}, {256, 74, "IQ2_XS"}, {256, 98, "IQ3_XXS"}, {256, 50, "IQ1_S"},
    {32, 18, "IQ4_NL"}, {256, 110, "IQ3_S"}, {256, 82, "IQ2_S"},  {256, 136, "IQ4_XS"}, {1, 1, "I8"},
    {1, 2, "I16"},      {1, 4, "I32"},       {1, 8, "I64"},       {1, 8, "F64"},      {256, 56, "IQ1_M"},
    {1, 2, "BF16"},     {0, 0, nullptr},     {0, 0, nullptr},     {0, 0, nullptr},    {256, 54, "TQ1_0"},
    {256, 66, "TQ2_0"}, {0, 0, nullptr},     {0, 0, nullptr},     {0, 0, nullptr},    {32, 17, "MXFP4"},
};

const TypeSize *type_size(uint32_t t) { return t < N_TYPES && TYPES[t].elems ? &TYPES[t] : nullptr; }

// Bytes of a fixed-size metadata value, 0 for STRING, ARRAY and unknown types.
uint32_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case RRR_GGUF_UINT8: case RRR_GGUF_INT8: case RRR_GGUF_BOOL: return 1;
    case RRR_GGUF_UINT16: case RRR_GGUF_INT16: return 2;
    case RRR_GGUF_UINT32: case RRR_GGUF_INT32: case RRR_GGUF_FLOAT32: return 4;
    case RRR_GGUF_UINT64: case RRR_GGUF_INT64: case RRR_GGUF_FLOAT64: return 8;
    default: return 0;
    }
}

bool utf8_valid(const uint8_t *s, uint64_t n)
{
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) { ++i; continue; }
        uint32_t len, cp;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (n - i < len) return false;
        for (uint32_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = cp << 6 | (s[i + k] & 0x3F);
        }
        const uint32_t min_cp = len == 2 ? 0x80 : len == 3 ? 0x800 : 0x10000;
        if (cp < min_cp || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

// Sequential reader over the image; every read checks the remaining length.
struct Cursor {
    const uint8_t *p;
    uint64_t size, pos;

    uint64_t left() const { return size - pos; }
    template <class T> bool get(T *v)
    {
        if (sizeof(T) > left()) return false;
        std::memcpy(v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool skip(uint64_t n)
    {
        if (n > left()) return false;
        pos += n;
        return true;
    }
};

int past_end(const Cursor &c, const char *what, const std::string &owner)
{
    return err(RRR_ERR_FORMAT, "%s%s%s runs past the end of the file (at byte %llu of %llu)", what,
               owner.empty() ? "" : " of ", owner.c_str(), (ull)c.pos, (ull)c.size);
}

// A length-prefixed string; sets *off to its first byte and *len.
int read_string(Cursor &c, uint64_t *off, uint64_t *len, const char *what, const std::string &owner)
{
    if (!c.get(len)) return past_end(c, what, owner);
    *off = c.pos;
    if (!c.skip(*len)) {
        c.pos -= 8;
        return err(RRR_ERR_FORMAT, "%s%s%s: length %llu at byte %llu runs past the end of the file (%llu bytes)",
                   what, owner.empty() ? "" : " of ", owner.c_str(), (ull)*len, (ull)c.pos, (ull)c.size);
    }
    return RRR_OK;
}

// Skips one value of `type`, validating it; `strs` (top-level string arrays)
// collects each element's record offset.
int read_value(Cursor &c, uint32_t type, int depth, const std::string &key, std::vector<uint64_t> *strs)
{
    if (uint32_t n = scalar_bytes(type)) {
        if (!c.skip(n)) return past_end(c, "value", "key '" + key + "'");
        return RRR_OK;
    }
    if (type == RRR_GGUF_STRING) {
        uint64_t off, len;
        return read_string(c, &off, &len, "string value", "key '" + key + "'");
    }
    if (type != RRR_GGUF_ARRAY)
        return err(RRR_ERR_FORMAT, "key '%s': unknown value type %u at byte %llu", key.c_str(), type,
                   (ull)(c.pos - 4));
    if (depth >= MAX_ARRAY_DEPTH)
        return err(RRR_ERR_FORMAT, "key '%s': arrays nested deeper than %d", key.c_str(), MAX_ARRAY_DEPTH);
    uint32_t et;
    uint64_t n;
    if (!c.get(&et) || !c.get(&n)) return past_end(c, "array header", "key '" + key + "'");
    if (uint32_t eb = scalar_bytes(et)) {
        if (n > c.left() / eb)
            return err(RRR_ERR_FORMAT, "key '%s': %llu elements of %u bytes run past the end of the file",
                       key.c_str(), (ull)n, eb);
        c.pos += n * eb;
        return RRR_OK;
    }
    if (et != RRR_GGUF_STRING && et != RRR_GGUF_ARRAY)
        return err(RRR_ERR_FORMAT, "key '%s': unknown array element type %u", key.c_str(), et);
    // Every string element takes at least its 8-byte length, every array
    // element its 12-byte header: bound the count before looping over it.
    const uint64_t min_rec = et == RRR_GGUF_STRING ? 8 : 12;
    if (n > c.left() / min_rec)
        return err(RRR_ERR_FORMAT, "key '%s': %llu array elements cannot fit in the remaining %llu bytes",
                   key.c_str(), (ull)n, (ull)c.left());
    if (strs && et == RRR_GGUF_STRING) strs->reserve(n);
    for (uint64_t i = 0; i < n; ++i) {
        if (strs && et == RRR_GGUF_STRING) strs->push_back(c.pos);
        if (int rc = read_value(c, et, depth + 1, key, nullptr)) return rc;
    }
    return RRR_OK;
}

bool is_integer(uint32_t t)
{
    return t <= RRR_GGUF_INT32 || t == RRR_GGUF_UINT64 || t == RRR_GGUF_INT64;
}

// Integer value of a scalar kv, sign-extended; *neg set for a negative one.
uint64_t int_value(const rrr_gguf &g, const rrr_gguf::Kv &kv, bool *neg)
{
    const uint8_t *p = g.base + kv.off;
    int64_t s = 0;
    uint64_t u = 0;
    bool is_signed = true;
    switch (kv.type) {
    case RRR_GGUF_UINT8: u = p[0]; is_signed = false; break;
    case RRR_GGUF_INT8: s = (int8_t)p[0]; break;
    case RRR_GGUF_UINT16: { uint16_t v; std::memcpy(&v, p, 2); u = v; is_signed = false; break; }
    case RRR_GGUF_INT16: { int16_t v; std::memcpy(&v, p, 2); s = v; break; }
    case RRR_GGUF_UINT32: { uint32_t v; std::memcpy(&v, p, 4); u = v; is_signed = false; break; }
    case RRR_GGUF_INT32: { int32_t v; std::memcpy(&v, p, 4); s = v; break; }
    case RRR_GGUF_UINT64: std::memcpy(&u, p, 8); is_signed = false; break;
    default: std::memcpy(&s, p, 8); break;  // INT64
    }
    *neg = is_signed && s < 0;
    return is_signed ? (uint64_t)s : u;
}

int parse(rrr_gguf &g)
{
    Cursor c{g.base, g.size, 0};
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!c.get(&magic)) return err(RRR_ERR_FORMAT, "file of %llu bytes is too short for a GGUF header", (ull)g.size);
    if (magic != GGUF_MAGIC) return err(RRR_ERR_FORMAT, "not a GGUF file (magic 0x%08x)", magic);
    if (!c.get(&g.version)) return past_end(c, "version", "");
    if (g.version == 1) return err(RRR_ERR_FORMAT, "GGUF version 1 (32-bit counts) is not supported");
    if (g.version != 2 && g.version != 3) {
        const uint32_t v = __builtin_bswap32(g.version);
        if (v == 2 || v == 3) return err(RRR_ERR_FORMAT, "big-endian GGUF (version %u byte-swapped) is not supported", v);
        return err(RRR_ERR_FORMAT, "unsupported GGUF version %u", g.version);
    }
    if (!c.get(&n_tensors) || !c.get(&n_kv)) return past_end(c, "header counts", "");

    // key length (8) + value type (4) + at least one value byte
    if (n_kv > c.left() / 13)
        return err(RRR_ERR_FORMAT, "%llu metadata pairs cannot fit in the remaining %llu bytes", (ull)n_kv,
                   (ull)c.left());
    g.kvs.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        rrr_gguf::Kv kv;
        uint64_t koff, klen;
        if (int rc = read_string(c, &koff, &klen, "metadata key", "pair " + std::to_string(i))) return rc;
        if (!utf8_valid(g.base + koff, klen))
            return err(RRR_ERR_FORMAT, "metadata key %llu at byte %llu is not UTF-8", (ull)i, (ull)koff);
        kv.key.assign((const char *)g.base + koff, klen);
        if (kv.key.find('\0') != std::string::npos)
            return err(RRR_ERR_FORMAT, "metadata key %llu holds a NUL byte", (ull)i);
        if (!c.get(&kv.type)) return past_end(c, "value type", "key '" + kv.key + "'");
        const uint64_t start = c.pos;
        if (int rc = read_value(c, kv.type, 0, kv.key, &kv.strs)) return rc;
        kv.elem_type = kv.type;
        kv.off = start;
        kv.bytes = c.pos - start;
        kv.count = 1;
        if (kv.type == RRR_GGUF_STRING) {
            std::memcpy(&kv.count, g.base + start, 8);
            kv.off = start + 8;
            kv.bytes = kv.count;
        } else if (kv.type == RRR_GGUF_ARRAY) {
            std::memcpy(&kv.elem_type, g.base + start, 4);
            std::memcpy(&kv.count, g.base + start + 4, 8);
            kv.off = start + 12;
            kv.bytes = c.pos - kv.off;
        }
        if (!g.kv_index.emplace(kv.key, g.kvs.size()).second)
            return err(RRR_ERR_FORMAT, "duplicate metadata key '%s'", kv.key.c_str());
        g.kvs.push_back(std::move(kv));
    }

    // name length (8) + n_dims (4) + type (4) + offset (8)
    if (n_tensors > c.left() / 24)
        return err(RRR_ERR_FORMAT, "%llu tensor records cannot fit in the remaining %llu bytes", (ull)n_tensors,
                   (ull)c.left());
    g.tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        rrr_gguf::Tensor t;
        uint64_t noff, nlen;
        if (int rc = read_string(c, &noff, &nlen, "tensor name", "tensor " + std::to_string(i))) return rc;
        if (!utf8_valid(g.base + noff, nlen))
            return err(RRR_ERR_FORMAT, "tensor name %llu at byte %llu is not UTF-8", (ull)i, (ull)noff);
        t.name.assign((const char *)g.base + noff, nlen);
        if (t.name.find('\0') != std::string::npos)
            return err(RRR_ERR_FORMAT, "tensor name %llu holds a NUL byte", (ull)i);
        const std::string who = "tensor '" + t.name + "'";
        if (!c.get(&t.n_dims)) return past_end(c, "dimension count", who);
        if (t.n_dims > 4) return err(RRR_ERR_FORMAT, "%s has %u dimensions (at most 4)", who.c_str(), t.n_dims);
        t.n_elements = 1;
        for (uint32_t d = 0; d < 4; ++d) {
            t.dims[d] = 1;
            if (d < t.n_dims) {
                if (!c.get(&t.dims[d])) return past_end(c, "dimensions", who);
                if (t.dims[d] > (uint64_t)INT64_MAX ||
                    __builtin_mul_overflow(t.n_elements, t.dims[d], &t.n_elements) || t.n_elements > (uint64_t)INT64_MAX)
                    return err(RRR_ERR_FORMAT, "%s: element count overflows 63 bits", who.c_str());
            }
        }
        if (!c.get(&t.type) || !c.get(&t.offset)) return past_end(c, "type and offset", who);
        const TypeSize *ts = type_size(t.type);
        if (!ts) return err(RRR_ERR_FORMAT, "%s has unknown ggml type %u", who.c_str(), t.type);
        if (t.dims[0] % ts->elems)
            return err(RRR_ERR_FORMAT, "%s: row length ne0=%llu is not a multiple of the %u-element %s block",
                       who.c_str(), (ull)t.dims[0], ts->elems, ts->name);
        if (__builtin_mul_overflow(t.n_elements / ts->elems, (uint64_t)ts->bytes, &t.bytes))
            return err(RRR_ERR_FORMAT, "%s: byte size overflows 64 bits", who.c_str());
        if (!g.tensor_index.emplace(t.name, g.tensors.size()).second)
            return err(RRR_ERR_FORMAT, "duplicate tensor name '%s'", t.name.c_str());
        g.tensors.push_back(std::move(t));
    }

    g.alignment = 32;  // the specification's default (gguf.rs:162)
    auto it = g.kv_index.find("general.alignment");
    if (it != g.kv_index.end()) {
        const rrr_gguf::Kv &kv = g.kvs[it->second];
        if (!is_integer(kv.type))
            return err(RRR_ERR_FORMAT, "general.alignment has value type %u, not an integer", kv.type);
        bool neg;
        const uint64_t a = int_value(g, kv, &neg);
        if (neg || a == 0 || (a & (a - 1)) || a > MAX_ALIGNMENT)
            return err(RRR_ERR_FORMAT, "general.alignment=%lld is not a power of two in [1, 2^30]", (long long)a);
        g.alignment = a;
    }
    g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
    const uint64_t avail = g.size > g.data_offset ? g.size - g.data_offset : 0;
    for (const rrr_gguf::Tensor &t : g.tensors) {
        if (t.offset % g.alignment)
            return err(RRR_ERR_FORMAT, "tensor '%s': offset %llu is not a multiple of the alignment %llu",
                       t.name.c_str(), (ull)t.offset, (ull)g.alignment);
        if (t.offset > avail || t.bytes > avail - t.offset)
            return err(RRR_ERR_FORMAT,
                       "tensor '%s': %llu bytes at data offset %llu run past the end of the file (data section "
                       "%llu bytes from byte %llu)",
                       t.name.c_str(), (ull)t.bytes, (ull)t.offset, (ull)avail, (ull)g.data_offset);
    }
    return RRR_OK;
}

int open_image(rrr_gguf *g, rrr_gguf **out)
{
    g->magic = HANDLE_MAGIC;
    if (int rc = parse(*g)) {
        if (g->mapped) munmap((void *)g->base, g->size);
        delete g;
        return rc;
    }
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_live.insert(g);
    }
    *out = g;
    return ok();
}

int check(const rrr_gguf *g)
{
    if (!g) return err(RRR_ERR_NULL, "null GGUF handle");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_live.count(g) || g->magic != HANDLE_MAGIC) return err(RRR_ERR_STALE, "GGUF handle already closed");
    return RRR_OK;
}

void fill_kv(const rrr_gguf &g, const rrr_gguf::Kv &kv, rrr_gguf_kv *out)
{
    out->key = kv.key.c_str();
    out->key_len = kv.key.size();
    out->type = kv.type;
    out->elem_type = kv.elem_type;
    out->count = kv.count;
    out->data = g.base + kv.off;
    out->bytes = kv.bytes;
}

void fill_tensor(const rrr_gguf &g, const rrr_gguf::Tensor &t, rrr_gguf_tensor *out)
{
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->n_dims = t.n_dims;
    out->type = t.type;
    std::memcpy(out->dims, t.dims, sizeof t.dims);
    out->offset = t.offset;
    out->n_elements = t.n_elements;
    out->bytes = t.bytes;
    out->data = t.bytes ? g.base + g.data_offset + t.offset : nullptr;
}

int lookup_kv(const rrr_gguf *g, const char *key, const rrr_gguf::Kv **kv)
{
    if (int rc = check(g)) return rc;
    if (!key) return err(RRR_ERR_NULL, "null key");
    auto it = g->kv_index.find(key);
    if (it == g->kv_index.end()) return err(RRR_ERR_NOT_FOUND, "no metadata key '%s'", key);
    *kv = &g->kvs[it->second];
    return RRR_OK;
}

}  // namespace

extern "C" {

int rrr_gguf_open(const char *path, rrr_gguf **out)
{
    if (!out) return err(RRR_ERR_NULL, "rrr_gguf_open: null output pointer");
    *out = nullptr;
    if (!path) return err(RRR_ERR_NULL, "rrr_gguf_open: null path");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return err(RRR_ERR_IO, "cannot open '%s': %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return err(RRR_ERR_IO, "cannot stat '%s': %s", path, strerror(e));
    }
    if (!S_ISREG(st.st_mode)) {
        close(fd);
        return err(RRR_ERR_IO, "'%s' is not a regular file", path);
    }
    if (st.st_size == 0) {
        close(fd);
        return err(RRR_ERR_FORMAT, "'%s' is empty", path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    close(fd);
    if (m == MAP_FAILED) return err(RRR_ERR_IO, "cannot map '%s': %s", path, strerror(e));
    rrr_gguf *g = new rrr_gguf();
    g->base = (const uint8_t *)m;
    g->size = (uint64_t)st.st_size;
    g->mapped = true;
    return open_image(g, out);
}

int rrr_gguf_open_memory(const void *data, uint64_t bytes, rrr_gguf **out)
{
    if (!out) return err(RRR_ERR_NULL, "rrr_gguf_open_memory: null output pointer");
    *out = nullptr;
    if (!data) return err(RRR_ERR_NULL, "rrr_gguf_open_memory: null data");
    rrr_gguf *g = new rrr_gguf();
    g->base = (const uint8_t *)data;
    g->size = bytes;
    g->mapped = false;
    return open_image(g, out);
}

int rrr_gguf_close(rrr_gguf *g)
{
    if (!g) return ok();
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_live.erase(g) || g->magic != HANDLE_MAGIC) return err(RRR_ERR_STALE, "GGUF handle already closed");
    }
    g->magic = 0;
    if (g->mapped) munmap((void *)g->base, g->size);
    delete g;
    return ok();
}

int rrr_gguf_header(const rrr_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv, uint64_t *alignment,
                    uint64_t *data_offset)
{
    if (int rc = check(g)) return rc;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kvs.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    return ok();
}

int rrr_gguf_kv_at(const rrr_gguf *g, uint64_t index, rrr_gguf_kv *out)
{
    if (int rc = check(g)) return rc;
    if (!out) return err(RRR_ERR_NULL, "rrr_gguf_kv_at: null output");
    if (index >= g->kvs.size())
        return err(RRR_ERR_INVALID_ARG, "metadata index %llu out of range (%llu pairs)", (ull)index,
                   (ull)g->kvs.size());
    fill_kv(*g, g->kvs[index], out);
    return ok();
}

int rrr_gguf_find_kv(const rrr_gguf *g, const char *key, uint64_t *index)
{
    const rrr_gguf::Kv *kv;
    if (int rc = lookup_kv(g, key, &kv)) return rc;
    if (!index) return err(RRR_ERR_NULL, "rrr_gguf_find_kv: null output");
    *index = (uint64_t)(kv - g->kvs.data());
    return ok();
}

int rrr_gguf_kv_strings(const rrr_gguf *g, uint64_t index, uint64_t first, uint64_t count, const char **ptrs,
                        uint64_t *lens)
{
    if (int rc = check(g)) return rc;
    if (index >= g->kvs.size())
        return err(RRR_ERR_INVALID_ARG, "metadata index %llu out of range (%llu pairs)", (ull)index,
                   (ull)g->kvs.size());
    if (count && (!ptrs || !lens)) return err(RRR_ERR_NULL, "rrr_gguf_kv_strings: null output arrays");
    const rrr_gguf::Kv &kv = g->kvs[index];
    if (kv.type == RRR_GGUF_STRING) {
        if (first > 1 || count > 1 - first)
            return err(RRR_ERR_INVALID_ARG, "key '%s' is one string; strings %llu..+%llu requested", kv.key.c_str(),
                       (ull)first, (ull)count);
        if (count) {
            ptrs[0] = (const char *)g->base + kv.off;
            lens[0] = kv.count;
        }
        return ok();
    }
    if (kv.type != RRR_GGUF_ARRAY || kv.elem_type != RRR_GGUF_STRING)
        return err(RRR_ERR_BAD_TYPE, "key '%s' is not a string or an array of strings", kv.key.c_str());
    if (first > kv.strs.size() || count > kv.strs.size() - first)
        return err(RRR_ERR_INVALID_ARG, "key '%s' holds %llu strings; %llu..+%llu requested", kv.key.c_str(),
                   (ull)kv.strs.size(), (ull)first, (ull)count);
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t rec = kv.strs[first + i];
        std::memcpy(&lens[i], g->base + rec, 8);
        ptrs[i] = (const char *)g->base + rec + 8;
    }
    return ok();
}

int rrr_gguf_get_u64(const rrr_gguf *g, const char *key, uint64_t *value)
{
    const rrr_gguf::Kv *kv;
    if (int rc = lookup_kv(g, key, &kv)) return rc;
    if (!value) return err(RRR_ERR_NULL, "rrr_gguf_get_u64: null output");
    if (!is_integer(kv->type)) return err(RRR_ERR_BAD_TYPE, "key '%s' has value type %u, not an integer", key, kv->type);
    bool neg;
    const uint64_t v = int_value(*g, *kv, &neg);
    if (neg) return err(RRR_ERR_INVALID_ARG, "key '%s' holds the negative value %lld", key, (long long)v);
    *value = v;
    return ok();
}

int rrr_gguf_get_f64(const rrr_gguf *g, const char *key, double *value)
{
    const rrr_gguf::Kv *kv;
    if (int rc = lookup_kv(g, key, &kv)) return rc;
    if (!value) return err(RRR_ERR_NULL, "rrr_gguf_get_f64: null output");
    if (kv->type == RRR_GGUF_FLOAT32) {
        float f;
        std::memcpy(&f, g->base + kv->off, 4);
        *value = f;
    } else if (kv->type == RRR_GGUF_FLOAT64) {
        std::memcpy(value, g->base + kv->off, 8);
    } else {
        return err(RRR_ERR_BAD_TYPE, "key '%s' has value type %u, not FLOAT32 or FLOAT64", key, kv->type);
    }
    return ok();
}

int rrr_gguf_get_str(const rrr_gguf *g, const char *key, const char **str, uint64_t *len)
{
    const rrr_gguf::Kv *kv;
    if (int rc = lookup_kv(g, key, &kv)) return rc;
    if (!str || !len) return err(RRR_ERR_NULL, "rrr_gguf_get_str: null output");
    if (kv->type != RRR_GGUF_STRING) return err(RRR_ERR_BAD_TYPE, "key '%s' has value type %u, not STRING", key, kv->type);
    *str = (const char *)g->base + kv->off;
    *len = kv->count;
    return ok();
}

int rrr_gguf_tensor_at(const rrr_gguf *g, uint64_t index, rrr_gguf_tensor *out)
{
    if (int rc = check(g)) return rc;
    if (!out) return err(RRR_ERR_NULL, "rrr_gguf_tensor_at: null output");
    if (index >= g->tensors.size())
        return err(RRR_ERR_INVALID_ARG, "tensor index %llu out of range (%llu tensors)", (ull)index,
                   (ull)g->tensors.size());
    fill_tensor(*g, g->tensors[index], out);
    return ok();
}

int rrr_gguf_find_tensor(const rrr_gguf *g, const char *name, rrr_gguf_tensor *out)
{
    if (int rc = check(g)) return rc;
    if (!name || !out) return err(RRR_ERR_NULL, "rrr_gguf_find_tensor: null name or output");
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return err(RRR_ERR_NOT_FOUND, "no tensor '%s'", name);
    fill_tensor(*g, g->tensors[it->second], out);
    return ok();
}

int rrr_gguf_type_size(uint32_t ggml_type, uint32_t *block_elems, uint32_t *block_bytes)
{
    const TypeSize *ts = type_size(ggml_type);
    if (!ts) return err(RRR_ERR_BAD_TYPE, "unknown ggml type %u", ggml_type);
    if (block_elems) *block_elems = ts->elems;
    if (block_bytes) *block_bytes = ts->bytes;
    return ok();
}

}  // extern "C"
