// GGUF v3 model files: read-only mapping, metadata and tensor directory,
// and the one-time upload of a tensor's bytes (native block layout, no
// repacking) into device memory.
//
// Follows SharpInference.Gguf/GgufModelFile.cs: magic and version (:79-80),
// count limits (:81-82, :303-306), metadata keys and values (:84-98,
// :201-255), legacy 32-bit array counts (:285-296), tensor descriptors
// (:100-119), general.alignment (:121-126), data start (:127), bounds of
// every tensor (:144-153) and byte lengths per type (:301-331).  Two
// departures, both widenings: the K-quant types (Q2_K..Q8_K, 256-element
// super-blocks) have byte lengths instead of being rejected (:320), and
// tensors of more than 2 GiB are addressable (the reference's Bytes span
// stops at int.MaxValue, :368-372).
#include "si_context.hpp"

#include <fcntl.h>
#include <stdarg.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

using namespace si_abi;

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;   // "GGUF"
constexpr uint32_t GGUF_VERSION = 3;
constexpr uint64_t COUNT_LIMIT = 0x7fffffffull;

enum ValueType : int {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

int scalar_size(int t)
{
    switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
    }
}

struct ParseError {
    int code;
    std::string message;
};

[[noreturn]] void bad(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw ParseError{code, buf};
}

// Strict UTF-8 (no overlong forms, no surrogates, nothing above U+10FFFF).
bool valid_utf8(const uint8_t* s, uint64_t n)
{
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t cp;
        if ((c & 0xe0) == 0xc0) { len = 2; cp = c & 0x1f; }
        else if ((c & 0xf0) == 0xe0) { len = 3; cp = c & 0x0f; }
        else if ((c & 0xf8) == 0xf0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n)
            return false;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xc0) != 0x80)
                return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) || cp > 0x10ffff ||
            (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += len;
    }
    return true;
}

struct Cursor {
    const uint8_t* p;
    uint64_t n;
    uint64_t at = 0;

    const uint8_t* take(uint64_t k)
    {
        if (k > n - at)
            bad(SI_HIP_ERR_FORMAT, "GGUF file is truncated at byte %llu", static_cast<unsigned long long>(at));
        const uint8_t* r = p + at;
        at += k;
        return r;
    }
    template <typename T>
    T get()
    {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str()
    {
        const uint64_t len = get<uint64_t>();
        if (len > COUNT_LIMIT)
            bad(SI_HIP_ERR_FORMAT, "GGUF string byte count %llu is too large", static_cast<unsigned long long>(len));
        const uint8_t* b = take(len);
        if (!valid_utf8(b, len))
            bad(SI_HIP_ERR_FORMAT, "GGUF string is not valid UTF-8");
        return std::string(reinterpret_cast<const char*>(b), len);
    }
};

struct Value {
    std::string key;
    int type = 0;
    int array_type = -1;
    uint64_t count = 1;
    std::vector<uint8_t> data;           // scalars and numeric arrays, native layout
    std::vector<std::string> strings;    // string value(s)
    std::vector<const char*> string_ptrs;
    std::vector<uint64_t> lengths;
};

struct Tensor {
    std::string name;
    int type = 0;
    int rank = 0;
    uint64_t dims[8] = {};
    uint64_t rel_offset = 0;
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

void read_elements(Cursor& c, Value& v, int t, uint64_t count)
{
    if (t == V_STRING) {
        for (uint64_t i = 0; i < count; i++)
            v.strings.push_back(c.str());
        return;
    }
    const int sz = scalar_size(t);
    if (sz == 0)
        bad(SI_HIP_ERR_FORMAT, "Unsupported GGUF %s type %d", v.array_type >= 0 ? "array" : "metadata", t);
    if (count > (c.n - c.at) / sz)
        bad(SI_HIP_ERR_FORMAT, "GGUF metadata '%s' is truncated", v.key.c_str());
    const uint8_t* b = c.take(count * sz);
    if (t == V_BOOL)
        for (uint64_t i = 0; i < count; i++)
            if (b[i] > 1)
                bad(SI_HIP_ERR_FORMAT, "Invalid GGUF Boolean value %d in '%s'", b[i], v.key.c_str());
    v.data.assign(b, b + count * sz);
}

// GgufModelFile.ReadArrayCount (:285-296): a count that does not fit a
// signed 32-bit int is read again as the 32-bit count older converters wrote.
uint64_t array_count(Cursor& c)
{
    const uint64_t v = c.get<uint64_t>();
    if (v <= COUNT_LIMIT)
        return v;
    const uint32_t legacy = static_cast<uint32_t>(v);
    if (legacy > COUNT_LIMIT)
        bad(SI_HIP_ERR_FORMAT, "GGUF array count %llu is too large", static_cast<unsigned long long>(v));
    c.at -= 4;
    return legacy;
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t* r)
{
    return !__builtin_mul_overflow(a, b, r);
}

// (elements per block, bytes per block) of a GGUF tensor type; {0, 0} for
// types without a byte length.
void type_layout(int type, uint64_t* be, uint64_t* bb)
{
    struct L { int t; uint64_t e, b; };
    static const L table[] = {
        {0, 1, 4}, {1, 1, 2}, {30, 1, 2}, {24, 1, 1}, {25, 1, 2}, {26, 1, 4}, {27, 1, 8}, {28, 1, 8},
        {2, 32, 18}, {3, 32, 20}, {6, 32, 22}, {7, 32, 24}, {8, 32, 34}, {9, 32, 36},
        {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292},
    };
    for (const L& l : table)
        if (l.t == type) {
            *be = l.e;
            *bb = l.b;
            return;
        }
    *be = *bb = 0;
}

}  // namespace

struct si_gguf {
    int fd = -1;
    void* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_start = 0;
    std::vector<Value> values;
    std::unordered_map<std::string, int64_t> value_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> tensor_index;

    ~si_gguf()
    {
        if (map && map != MAP_FAILED)
            munmap(map, size);
        if (fd >= 0)
            close(fd);
    }
};

namespace {

void parse(si_gguf* g)
{
    Cursor c{static_cast<const uint8_t*>(g->map), g->size};
    if (c.get<uint32_t>() != GGUF_MAGIC || (g->version = c.get<uint32_t>()) != GGUF_VERSION)
        bad(SI_HIP_ERR_FORMAT, "Expected a GGUF v3 model file.");
    const uint64_t tensor_count = c.get<uint64_t>();
    const uint64_t value_count = c.get<uint64_t>();
    if (tensor_count > COUNT_LIMIT)
        bad(SI_HIP_ERR_FORMAT, "GGUF tensor count %llu is too large.", static_cast<unsigned long long>(tensor_count));
    if (value_count > COUNT_LIMIT)
        bad(SI_HIP_ERR_FORMAT, "GGUF metadata count %llu is too large.", static_cast<unsigned long long>(value_count));

    for (uint64_t i = 0; i < value_count; i++) {
        Value v;
        v.key = c.str();
        bool blank = true;
        for (char ch : v.key)
            blank &= ch == ' ' || ch == '\t' || ch == '\n' || ch == '\r' || ch == '\v' || ch == '\f';
        if (blank || g->value_index.count(v.key))
            bad(SI_HIP_ERR_FORMAT, "Empty or duplicate GGUF metadata key '%s'.", v.key.c_str());
        v.type = static_cast<int>(c.get<uint32_t>());
        if (v.type == V_ARRAY) {
            v.array_type = static_cast<int>(c.get<uint32_t>());
            if (v.array_type == V_ARRAY)
                bad(SI_HIP_ERR_FORMAT, "Nested GGUF metadata arrays are unsupported ('%s').", v.key.c_str());
            v.count = array_count(c);
            read_elements(c, v, v.array_type, v.count);
        } else {
            read_elements(c, v, v.type, 1);
        }
        for (const std::string& s : v.strings) {
            v.string_ptrs.push_back(s.c_str());
            v.lengths.push_back(s.size());
        }
        g->value_index.emplace(v.key, static_cast<int64_t>(g->values.size()));
        g->values.push_back(std::move(v));
    }

    for (uint64_t i = 0; i < tensor_count; i++) {
        Tensor t;
        t.name = c.str();
        bool blank = true;
        for (char ch : t.name)
            blank &= ch == ' ' || ch == '\t' || ch == '\n' || ch == '\r' || ch == '\v' || ch == '\f';
        if (blank || g->tensor_index.count(t.name))
            bad(SI_HIP_ERR_FORMAT, "Empty or duplicate GGUF tensor name '%s'.", t.name.c_str());
        const uint32_t rank = c.get<uint32_t>();
        if (rank < 1 || rank > 8)
            bad(SI_HIP_ERR_FORMAT, "Tensor '%s' has unsupported rank %u.", t.name.c_str(), rank);
        t.rank = static_cast<int>(rank);
        for (uint32_t d = 0; d < rank; d++) {
            t.dims[d] = c.get<uint64_t>();
            if (t.dims[d] == 0)
                bad(SI_HIP_ERR_FORMAT, "Tensor '%s' has an empty dimension.", t.name.c_str());
        }
        t.type = static_cast<int>(c.get<uint32_t>());
        t.rel_offset = c.get<uint64_t>();
        g->tensor_index.emplace(t.name, static_cast<int64_t>(g->tensors.size()));
        g->tensors.push_back(std::move(t));
    }

    auto it = g->value_index.find("general.alignment");
    if (it != g->value_index.end()) {
        const Value& v = g->values[it->second];
        uint64_t a = 0;
        switch (v.type) {
        case V_U8: a = v.data[0]; break;
        case V_U16: { uint16_t x; std::memcpy(&x, v.data.data(), 2); a = x; break; }
        case V_U32: { uint32_t x; std::memcpy(&x, v.data.data(), 4); a = x; break; }
        case V_U64: std::memcpy(&a, v.data.data(), 8); break;
        case V_I8: case V_I16: case V_I32: case V_I64: {
            int64_t x = 0;
            if (v.type == V_I8) x = static_cast<int8_t>(v.data[0]);
            else if (v.type == V_I16) { int16_t y; std::memcpy(&y, v.data.data(), 2); x = y; }
            else if (v.type == V_I32) { int32_t y; std::memcpy(&y, v.data.data(), 4); x = y; }
            else std::memcpy(&x, v.data.data(), 8);
            if (x < 0)
                bad(SI_HIP_ERR_FORMAT, "Invalid GGUF alignment %lld.", static_cast<long long>(x));
            a = static_cast<uint64_t>(x);
            break;
        }
        default: bad(SI_HIP_ERR_FORMAT, "GGUF general.alignment is not an integer.");
        }
        if (a == 0 || a > 0xffffffffull || (a & (a - 1)) != 0)
            bad(SI_HIP_ERR_FORMAT, "Invalid GGUF alignment %llu.", static_cast<unsigned long long>(a));
        g->alignment = a;
    }
    g->data_start = (c.at + g->alignment - 1) & ~(g->alignment - 1);

    for (Tensor& t : g->tensors) {
        uint64_t elements = 1;
        for (int d = 0; d < t.rank; d++)
            if (!mul_ok(elements, t.dims[d], &elements))
                bad(SI_HIP_ERR_FORMAT, "Tensor '%s' has too many elements.", t.name.c_str());
        uint64_t be, bb;
        type_layout(t.type, &be, &bb);
        if (be == 0)
            bad(SI_HIP_ERR_UNSUPPORTED, "GGUF tensor type %d of '%s' is not supported.", t.type, t.name.c_str());
        if (elements % be != 0)
            bad(SI_HIP_ERR_FORMAT, "Quantized tensor element count %llu is not divisible by block size %llu.",
                static_cast<unsigned long long>(elements), static_cast<unsigned long long>(be));
        if (!mul_ok(elements / be, bb, &t.bytes))
            bad(SI_HIP_ERR_FORMAT, "Tensor '%s' is too large.", t.name.c_str());
        if (__builtin_add_overflow(g->data_start, t.rel_offset, &t.offset) || t.offset > g->size ||
            t.bytes > g->size - t.offset)
            bad(SI_HIP_ERR_FORMAT, "Tensor '%s' exceeds the GGUF file.", t.name.c_str());
    }
}

}  // namespace

extern "C" {

int si_gguf_open(const char* path, si_gguf** out)
{
    if (!path || !out)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_open: null argument");
    *out = nullptr;
    auto* g = new si_gguf();
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        const int err = errno;
        delete g;
        return fail(nullptr, SI_HIP_ERR_IO, "gguf_open: cannot open '%s': %s", path, strerror(err));
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        delete g;
        return fail(nullptr, SI_HIP_ERR_IO, "gguf_open: '%s' is not a regular file", path);
    }
    g->size = static_cast<uint64_t>(st.st_size);
    if (g->size < 24) {
        delete g;
        return fail(nullptr, SI_HIP_ERR_FORMAT, "gguf_open: Expected a GGUF v3 model file ('%s' has %llu bytes).",
                    path, static_cast<unsigned long long>(g->size));
    }
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        const int err = errno;
        g->map = nullptr;
        delete g;
        return fail(nullptr, SI_HIP_ERR_IO, "gguf_open: cannot map '%s': %s", path, strerror(err));
    }
    try {
        parse(g);
    } catch (const ParseError& e) {
        delete g;
        return fail(nullptr, e.code, "gguf_open: %s", e.message.c_str());
    } catch (const std::bad_alloc&) {
        delete g;
        return fail(nullptr, SI_HIP_ERR_OUT_OF_MEMORY, "gguf_open: out of host memory");
    }
    *out = g;
    return SI_HIP_OK;
}

int si_gguf_close(si_gguf* file)
{
    delete file;
    return SI_HIP_OK;
}

int si_gguf_info(const si_gguf* file, si_gguf_file_info* info)
{
    if (!file || !info)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_info: null argument");
    info->version = file->version;
    info->alignment = file->alignment;
    info->data_start = file->data_start;
    info->file_bytes = file->size;
    info->tensor_count = static_cast<int64_t>(file->tensors.size());
    info->metadata_count = static_cast<int64_t>(file->values.size());
    return SI_HIP_OK;
}

int si_gguf_tensor_at(const si_gguf* file, int64_t index, si_gguf_tensor* out)
{
    if (!file || !out)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_tensor_at: null argument");
    if (index < 0 || index >= static_cast<int64_t>(file->tensors.size()))
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_tensor_at: index %lld outside 0..%lld",
                    static_cast<long long>(index), static_cast<long long>(file->tensors.size()) - 1);
    const Tensor& t = file->tensors[index];
    out->name = t.name.c_str();
    out->type = t.type;
    out->rank = t.rank;
    for (int d = 0; d < 8; d++)
        out->dims[d] = d < t.rank ? t.dims[d] : 1;
    out->offset = t.offset;
    out->bytes = t.bytes;
    out->data = static_cast<const uint8_t*>(file->map) + t.offset;
    return SI_HIP_OK;
}

int si_gguf_find_tensor(const si_gguf* file, const char* name, int64_t* index)
{
    if (!file || !name || !index)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_find_tensor: null argument");
    auto it = file->tensor_index.find(name);
    *index = it == file->tensor_index.end() ? -1 : it->second;
    return SI_HIP_OK;
}

int si_gguf_metadata_at(const si_gguf* file, int64_t index, si_gguf_value* out)
{
    if (!file || !out)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_metadata_at: null argument");
    if (index < 0 || index >= static_cast<int64_t>(file->values.size()))
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_metadata_at: index %lld outside 0..%lld",
                    static_cast<long long>(index), static_cast<long long>(file->values.size()) - 1);
    const Value& v = file->values[index];
    out->key = v.key.c_str();
    out->type = v.type;
    out->array_type = v.array_type;
    out->count = v.count;
    const bool strings = v.type == V_STRING || v.array_type == V_STRING;
    out->data = strings ? static_cast<const void*>(v.string_ptrs.data()) : static_cast<const void*>(v.data.data());
    out->lengths = strings ? v.lengths.data() : nullptr;
    return SI_HIP_OK;
}

int si_gguf_find_metadata(const si_gguf* file, const char* key, int64_t* index)
{
    if (!file || !key || !index)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_find_metadata: null argument");
    auto it = file->value_index.find(key);
    *index = it == file->value_index.end() ? -1 : it->second;
    return SI_HIP_OK;
}

int si_gguf_upload(si_hip_context* ctx, const si_gguf* file, int64_t index, void* device_dst, uint64_t dst_bytes)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gguf_upload: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "gguf_upload: not allowed while recording a plan");
    if (!file || !device_dst)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gguf_upload: null argument");
    if (index < 0 || index >= static_cast<int64_t>(file->tensors.size()))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gguf_upload: tensor index %lld out of range",
                    static_cast<long long>(index));
    const Tensor& t = file->tensors[index];
    if (dst_bytes < t.bytes)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gguf_upload: '%s' needs %llu bytes, destination has %llu",
                    t.name.c_str(), static_cast<unsigned long long>(t.bytes),
                    static_cast<unsigned long long>(dst_bytes));
    // the mapping pages in as the copy reads it; chunks keep each runtime
    // staging pass bounded
    const uint8_t* src = static_cast<const uint8_t*>(file->map) + t.offset;
    constexpr uint64_t CHUNK = 256ull << 20;
    hipError_t e = hipSuccess;
    for (uint64_t done = 0; e == hipSuccess && done < t.bytes; done += CHUNK) {
        const uint64_t n = t.bytes - done < CHUNK ? t.bytes - done : CHUNK;
        e = hipMemcpyAsync(static_cast<uint8_t*>(device_dst) + done, src + done, n, hipMemcpyHostToDevice,
                           ctx->stream);
    }
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gguf_upload");
}

}  // extern "C"
