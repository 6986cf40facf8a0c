// gguf.hip -- GGUF model files: parser, metadata queries, and the upload of
// all tensor data into one HBM arena (host code; no kernels).
//
// The accept/reject rules, the tensor table and the derived sizes follow the
// reference parser (src/ai/gguf.c) so that a file reads the same way in both;
// the citations are per rule below.  Two inputs crash the reference
// (a division by zero) and are given defined results here instead:
//   - tensor types 4, 5 and 16..23 have no block-size entry in the reference
//     table (gguf.c:50-71, divided by at gguf.c:106-109): size_bytes = 0 here;
//   - attention.head_count = 0 makes the default head dimension divide by
//     zero (gguf.c:383): attention_key_length defaults to 0 here.
#include "common.h"
#include "../../include/holo_gguf.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

namespace holo {
namespace {

constexpr uint32_t kMagic = 0x46554747u;           // "GGUF" little-endian (gguf.h:19)
constexpr uint64_t kMaxString = 1024ull * 1024ull;  // gguf.c:147
constexpr uint64_t kMaxArray = 10000000ull;         // gguf.c:202
constexpr uint32_t kMaxDims = 4;                    // gguf.h:73
constexpr uint64_t kDataAlign = 32;                 // gguf.c:355-356

// Bytes and elements per block of a GGML tensor type, as the reference's
// tables give them (gguf.c:26-71, GGML_TYPE_COUNT = 30): {0, 0} where the
// table has no entry, {0, 1} past its end.
struct TypeGeo {
    uint64_t bytes, block;
};

TypeGeo type_geo(uint32_t t)
{
    switch (t) {
    case 0: return {4, 1};       // F32
    case 1: return {2, 1};       // F16
    case 2: return {18, 32};     // Q4_0
    case 3: return {20, 32};     // Q4_1
    case 6: return {22, 32};     // Q5_0
    case 7: return {24, 32};     // Q5_1
    case 8: return {34, 32};     // Q8_0
    case 9: return {36, 32};     // Q8_1
    case 10: return {84, 256};   // Q2_K
    case 11: return {110, 256};  // Q3_K
    case 12: return {144, 256};  // Q4_K
    case 13: return {176, 256};  // Q5_K
    case 14: return {210, 256};  // Q6_K
    case 15: return {292, 256};  // Q8_K
    case 24: return {1, 1};      // I8
    case 25: return {2, 1};      // I16
    case 26: return {4, 1};      // I32
    case 27: return {8, 1};      // I64
    case 28: return {8, 1};      // F64
    case 29: return {2, 1};      // BF16
    default: return t < 30 ? TypeGeo{0, 0} : TypeGeo{0, 1};
    }
}

// ggml_row_size (gguf.c:106-109): whole blocks only, in signed 64-bit.
uint64_t tensor_bytes(uint32_t type, uint64_t n_elements)
{
    const TypeGeo g = type_geo(type);
    if (g.block == 0) return 0;
    return (uint64_t)(((int64_t)n_elements / (int64_t)g.block) * (int64_t)g.bytes);
}

uint64_t elem_bytes(uint32_t vt)
{
    switch (vt) {
    case HOLO_GGUF_UINT8: case HOLO_GGUF_INT8: case HOLO_GGUF_BOOL: return 1;
    case HOLO_GGUF_UINT16: case HOLO_GGUF_INT16: return 2;
    case HOLO_GGUF_UINT32: case HOLO_GGUF_INT32: case HOLO_GGUF_FLOAT32: return 4;
    case HOLO_GGUF_UINT64: case HOLO_GGUF_INT64: case HOLO_GGUF_FLOAT64: return 8;
    default: return 0;
    }
}

struct Value {
    uint32_t type = 0;
    union {
        uint8_t u8;
        int8_t i8;
        uint16_t u16;
        int16_t i16;
        uint32_t u32;
        int32_t i32;
        uint64_t u64;
        int64_t i64;
        float f32;
        double f64;
        bool b;
    } s{};
    std::string str;                          // STRING
    uint32_t arr_type = 0;                    // ARRAY: element type, count, data
    uint64_t arr_len = 0;
    std::vector<uint8_t> arr_raw;             // scalar elements, as in the file
    std::vector<std::string> arr_str;         // string elements
    std::vector<holo_gguf_string_t> arr_view; // {len, data} views of arr_str
};

struct Kv {
    std::string key;
    Value value;
};

// Sequential reader over the file's header region (buffered stdio).
struct Reader {
    FILE *f;
    bool get(void *p, size_t n) { return n == 0 || fread(p, 1, n, f) == n; }
    template <class T>
    bool pod(T &v) { return get(&v, sizeof(T)); }
    bool string(std::string &out)
    {
        uint64_t len = 0;
        if (!pod(len) || len > kMaxString) return false;
        out.resize((size_t)len);
        return get(&out[0], (size_t)len);
    }
};

bool read_value(Reader &r, Value &v)
{
    if (!r.pod(v.type)) return false;
    switch (v.type) {
    case HOLO_GGUF_UINT8: return r.pod(v.s.u8);
    case HOLO_GGUF_INT8: return r.pod(v.s.i8);
    case HOLO_GGUF_UINT16: return r.pod(v.s.u16);
    case HOLO_GGUF_INT16: return r.pod(v.s.i16);
    case HOLO_GGUF_UINT32: return r.pod(v.s.u32);
    case HOLO_GGUF_INT32: return r.pod(v.s.i32);
    case HOLO_GGUF_UINT64: return r.pod(v.s.u64);
    case HOLO_GGUF_INT64: return r.pod(v.s.i64);
    case HOLO_GGUF_FLOAT32: return r.pod(v.s.f32);
    case HOLO_GGUF_FLOAT64: return r.pod(v.s.f64);
    case HOLO_GGUF_BOOL: {
        uint8_t b = 0;
        if (!r.pod(b)) return false;
        v.s.b = b != 0;
        return true;
    }
    case HOLO_GGUF_STRING: return r.string(v.str);
    case HOLO_GGUF_ARRAY: {
        if (!r.pod(v.arr_type) || !r.pod(v.arr_len) || v.arr_len > kMaxArray) return false;
        if (v.arr_type == HOLO_GGUF_STRING) {
            v.arr_str.resize((size_t)v.arr_len);
            for (auto &e : v.arr_str)
                if (!r.string(e)) return false;
            v.arr_view.resize(v.arr_str.size());
            for (size_t i = 0; i < v.arr_str.size(); i++)
                v.arr_view[i] = {(uint64_t)v.arr_str[i].size(), &v.arr_str[i][0]};
            return true;
        }
        const uint64_t eb = elem_bytes(v.arr_type);
        if (eb == 0) return false;  // nested arrays and unknown types (gguf.c:228-229)
        v.arr_raw.resize((size_t)(eb * v.arr_len));
        return r.get(v.arr_raw.data(), v.arr_raw.size());
    }
    default: return false;
    }
}

}  // namespace
}  // namespace holo

struct holo_gguf {
    FILE *f = nullptr;
    uint32_t version = 0;
    std::vector<holo::Kv> kv;
    std::vector<holo_gguf_tensor_t> tensors;
    uint64_t data_offset = 0;
    holo_gguf_model_t model{};
    void *arena = nullptr;
    size_t arena_bytes = 0;
};

using namespace holo;

namespace {

const Value *find_value(const holo_gguf_t *g, const char *key)
{
    if (!g || !key) return nullptr;
    for (const auto &e : g->kv)
        if (strcmp(e.key.c_str(), key) == 0) return &e.value;  // first match, C-string compare (gguf.c:435-438)
    return nullptr;
}

// Model parameters: the reference's keys and defaults (gguf.c:358-393).
void read_model(holo_gguf_t *g)
{
    holo_gguf_model_t &m = g->model;
    const char *arch = holo_gguf_get_string(g, "general.architecture");
    if (arch) strncpy(m.arch, arch, sizeof(m.arch) - 1);
    char key[256];
    auto geti = [&](const char *suffix, int64_t def) {
        snprintf(key, sizeof(key), "%s.%s", m.arch, suffix);
        return (uint32_t)holo_gguf_get_int(g, key, def);
    };
    auto getf = [&](const char *suffix, float def) {
        snprintf(key, sizeof(key), "%s.%s", m.arch, suffix);
        return holo_gguf_get_float(g, key, def);
    };
    m.vocab_size = geti("vocab_size", 32000);
    m.context_length = geti("context_length", 4096);
    m.embedding_length = geti("embedding_length", 4096);
    m.block_count = geti("block_count", 32);
    m.attention_head_count = geti("attention.head_count", 32);
    m.attention_head_count_kv = geti("attention.head_count_kv", m.attention_head_count);
    const uint32_t head_dim = m.attention_head_count ? m.embedding_length / m.attention_head_count : 0;
    m.attention_key_length = geti("attention.key_length", head_dim);
    m.feed_forward_length = geti("feed_forward_length", 11008);
    m.rope_freq_base = getf("rope.freq_base", 10000.0f);
    m.rms_norm_eps = getf("attention.layer_norm_rms_epsilon", 1e-5f);
}

bool parse(holo_gguf_t *g)
{
    Reader r{g->f};
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.pod(magic) || magic != kMagic) {
        fprintf(stderr, "GGUF: Invalid magic number\n");
        return false;
    }
    if (!r.pod(g->version)) {
        fprintf(stderr, "GGUF: Cannot read version\n");
        return false;
    }
    if (g->version < 2 || g->version > 3) {
        fprintf(stderr, "GGUF: Unsupported version %u (need 2 or 3)\n", g->version);
        return false;
    }
    if (!r.pod(n_tensors) || !r.pod(n_kv)) {
        fprintf(stderr, "GGUF: Cannot read counts\n");
        return false;
    }
    // entries are read one by one, so a corrupt count fails on the first
    // missing entry instead of reserving memory for it
    for (uint64_t i = 0; i < n_kv; i++) {
        Kv e;
        if (!r.string(e.key)) {
            fprintf(stderr, "GGUF: Cannot read key %llu\n", (unsigned long long)i);
            return false;
        }
        if (!read_value(r, e.value)) {
            fprintf(stderr, "GGUF: Cannot read value for key '%s'\n", e.key.c_str());
            return false;
        }
        g->kv.push_back(std::move(e));
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        holo_gguf_tensor_t t;
        memset(&t, 0, sizeof(t));
        std::string name;
        if (!r.string(name)) return false;
        strncpy(t.name, name.c_str(), sizeof(t.name) - 1);
        if (!r.pod(t.n_dims) || t.n_dims > kMaxDims) return false;
        t.n_elements = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if (!r.pod(t.dims[d])) return false;
            t.n_elements *= t.dims[d];
        }
        uint32_t type = 0;
        if (!r.pod(type) || !r.pod(t.offset)) return false;
        t.type = (int32_t)type;
        t.size_bytes = tensor_bytes(type, t.n_elements);
        g->tensors.push_back(t);
    }
    const long pos = ftell(g->f);
    if (pos < 0) return false;
    g->data_offset = ((uint64_t)pos + kDataAlign - 1) & ~(kDataAlign - 1);
    read_model(g);
    return true;
}

// Reads n bytes at file offset off (pread loop).
bool read_at(FILE *f, void *dst, size_t n, uint64_t off)
{
    const int fd = fileno(f);
    uint8_t *p = (uint8_t *)dst;
    while (n > 0) {
        const ssize_t k = pread(fd, p, n, (off_t)off);
        if (k <= 0) return false;
        p += k;
        n -= (size_t)k;
        off += (uint64_t)k;
    }
    return true;
}

}  // namespace

extern "C" {

holo_gguf_t *holo_gguf_open(const char *path)
{
    if (!path) return nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "GGUF: Cannot open file: %s\n", path);
        return nullptr;
    }
    holo_gguf_t *g = new holo_gguf_t;
    g->f = f;
    if (!parse(g)) {
        holo_gguf_close(g);
        return nullptr;
    }
    return g;
}

void holo_gguf_close(holo_gguf_t *g)
{
    if (!g) return;
    if (g->arena) HOLO_CHECK(hipFree(g->arena));
    if (g->f) fclose(g->f);
    delete g;
}

uint32_t holo_gguf_version(const holo_gguf_t *g) { return g ? g->version : 0; }
uint64_t holo_gguf_n_tensors(const holo_gguf_t *g) { return g ? g->tensors.size() : 0; }
uint64_t holo_gguf_n_kv(const holo_gguf_t *g) { return g ? g->kv.size() : 0; }
uint64_t holo_gguf_data_offset(const holo_gguf_t *g) { return g ? g->data_offset : 0; }
const holo_gguf_model_t *holo_gguf_model(const holo_gguf_t *g) { return g ? &g->model : nullptr; }

const char *holo_gguf_key(const holo_gguf_t *g, uint64_t i)
{
    return g && i < g->kv.size() ? g->kv[i].key.c_str() : nullptr;
}

int holo_gguf_value_type(const holo_gguf_t *g, const char *key)
{
    const Value *v = find_value(g, key);
    return v ? (int)v->type : -1;
}

const char *holo_gguf_get_string(const holo_gguf_t *g, const char *key)
{
    const Value *v = find_value(g, key);
    return v && v->type == HOLO_GGUF_STRING ? v->str.c_str() : nullptr;
}

int64_t holo_gguf_get_int(const holo_gguf_t *g, const char *key, int64_t default_val)
{
    const Value *v = find_value(g, key);
    if (!v) return default_val;
    switch (v->type) {
    case HOLO_GGUF_UINT8: return v->s.u8;
    case HOLO_GGUF_INT8: return v->s.i8;
    case HOLO_GGUF_UINT16: return v->s.u16;
    case HOLO_GGUF_INT16: return v->s.i16;
    case HOLO_GGUF_UINT32: return v->s.u32;
    case HOLO_GGUF_INT32: return v->s.i32;
    case HOLO_GGUF_UINT64: return (int64_t)v->s.u64;
    case HOLO_GGUF_INT64: return v->s.i64;
    default: return default_val;
    }
}

float holo_gguf_get_float(const holo_gguf_t *g, const char *key, float default_val)
{
    const Value *v = find_value(g, key);
    if (!v) return default_val;
    if (v->type == HOLO_GGUF_FLOAT32) return v->s.f32;
    if (v->type == HOLO_GGUF_FLOAT64) return (float)v->s.f64;
    return default_val;
}

const void *holo_gguf_get_array(const holo_gguf_t *g, const char *key, uint64_t *len, int *elem_type)
{
    const Value *v = find_value(g, key);
    if (!v || v->type != HOLO_GGUF_ARRAY) {
        if (len) *len = 0;
        return nullptr;
    }
    if (len) *len = v->arr_len;
    if (elem_type) *elem_type = (int)v->arr_type;
    // an empty array is present: a valid pointer to no elements, as in
    // gguf.c:235-236 (malloc of zero bytes)
    static const uint64_t kNoElements = 0;
    if (v->arr_len == 0) return &kNoElements;
    if (v->arr_type == HOLO_GGUF_STRING) return v->arr_view.data();
    return v->arr_raw.data();
}

const holo_gguf_tensor_t *holo_gguf_tensor(const holo_gguf_t *g, uint64_t i)
{
    return g && i < g->tensors.size() ? &g->tensors[i] : nullptr;
}

const holo_gguf_tensor_t *holo_gguf_find_tensor(const holo_gguf_t *g, const char *name)
{
    if (!g || !name) return nullptr;
    for (const auto &t : g->tensors)
        if (strcmp(t.name, name) == 0) return &t;
    return nullptr;
}

int holo_gguf_load_tensor(holo_gguf_t *g, const holo_gguf_tensor_t *t, void *buffer, size_t size)
{
    if (!g || !t || !buffer || size < t->size_bytes) return -1;
    return read_at(g->f, buffer, (size_t)t->size_bytes, g->data_offset + t->offset) ? 0 : -1;
}

int holo_gguf_upload(holo_gguf_t *g)
{
    if (!g) return -1;
    if (g->arena) return 0;
    uint64_t end = 0;
    for (const auto &t : g->tensors) end = t.offset + t.size_bytes > end ? t.offset + t.size_bytes : end;
    if (end == 0) return 0;
    struct stat st;
    if (fstat(fileno(g->f), &st) != 0 || g->data_offset + end > (uint64_t)st.st_size) {
        fprintf(stderr, "GGUF: tensor data extends past the end of the file\n");
        return -1;
    }
    void *arena = nullptr;
    if (hipMalloc(&arena, (size_t)end) != hipSuccess || !arena) {
        (void)hipGetLastError();
        fprintf(stderr, "GGUF: cannot allocate %llu bytes of device memory\n", (unsigned long long)end);
        return -1;
    }
    // Two pinned staging buffers: the file read into one overlaps the copy
    // out of the other on the copy stream.
    const size_t chunk = (size_t)(end < (64ull << 20) ? end : (64ull << 20));
    void *pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t s = copy_stream() ? copy_stream() : stream();
    bool ok = true;
    for (int i = 0; i < 2 && ok; i++) {
        ok = hipHostMalloc(&pin[i], chunk, hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&done[i], hipEventDisableTiming) == hipSuccess;
    }
    uint64_t off = 0;
    for (int k = 0; ok && off < end; k++, off += chunk) {
        const int i = k & 1;
        const size_t n = (size_t)(end - off < chunk ? end - off : chunk);
        if (k >= 2) ok = hipEventSynchronize(done[i]) == hipSuccess;  // buffer i's previous copy is done
        ok = ok && read_at(g->f, pin[i], n, g->data_offset + off);
        ok = ok && hipMemcpyAsync((uint8_t *)arena + off, pin[i], n, hipMemcpyHostToDevice, s) == hipSuccess;
        ok = ok && hipEventRecord(done[i], s) == hipSuccess;
    }
    if (hipStreamSynchronize(s) != hipSuccess) ok = false;
    for (int i = 0; i < 2; i++) {
        if (pin[i]) HOLO_CHECK(hipHostFree(pin[i]));
        if (done[i]) HOLO_CHECK(hipEventDestroy(done[i]));
    }
    if (!ok) {
        (void)hipGetLastError();
        HOLO_CHECK(hipFree(arena));
        fprintf(stderr, "GGUF: upload failed\n");
        return -1;
    }
    g->arena = arena;
    g->arena_bytes = (size_t)end;
    return 0;
}

void *holo_gguf_device_base(const holo_gguf_t *g) { return g ? g->arena : nullptr; }
size_t holo_gguf_device_bytes(const holo_gguf_t *g) { return g ? g->arena_bytes : 0; }

void *holo_gguf_device_ptr(const holo_gguf_t *g, const holo_gguf_tensor_t *t)
{
    if (!g || !t || !g->arena) return nullptr;
    return (uint8_t *)g->arena + t->offset;
}

}  // extern "C"
