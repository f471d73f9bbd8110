// Checkpoints and weight formats: the safetensors reader and the device-side conversions that
// turn checkpoint tensors into the layouts the kernels read.
//
// Reader (Weights, crates/tts-nn/src/lib.rs:143-360): the file is memory-mapped read-only; its
// header -- an 8-byte little-endian length, then a JSON object mapping each name to
// {"dtype", "shape", "data_offsets": [begin, end]} relative to the byte buffer after the header,
// plus an optional "__metadata__" object -- is parsed once into a table. Offsets, sizes and
// dtype widths are checked against the file before any tensor is handed out.
//
// Conversions: one thread per destination element (grid-stride), reading the raw source in its
// on-disk dtype (f32, f16, bf16, f64) as f32 or f64. They run once per load and are HBM-bound
// passes; the transpose goes through a 32 x 33 LDS tile so both sides are coalesced.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

struct dtts_checkpoint {
    struct Entry {
        std::string name;
        int32_t dtype = DTTS_DT_OTHER;
        int32_t ndim = 0;
        int64_t shape[DTTS_TENSOR_MAX_DIMS] = {};
        size_t begin = 0, end = 0;
    };
    int fd = -1;
    void *map = nullptr;
    size_t size = 0;
    const char *data = nullptr;  // the byte buffer after the header
    size_t data_size = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> index;
};

namespace dtts {
namespace {

// ---------------------------------------------------------------- header JSON

// A strict reader for the subset of JSON a safetensors header is: objects, arrays, strings,
// integers (other numbers, true/false/null are accepted and skipped inside "__metadata__").
struct Json {
    const char *p, *end;
    std::string err;

    bool fail(const char *what) {
        if (err.empty()) err = what;
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool string(std::string &out) {
        ws();
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return fail("truncated escape");
                const char e = *p++;
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (end - p < 4) return fail("truncated \\u escape");
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= unsigned(h - '0');
                            else if (h >= 'a' && h <= 'f') v |= unsigned(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') v |= unsigned(h - 'A' + 10);
                            else return fail("bad \\u escape");
                        }
                        // UTF-8 of the code unit (surrogate pairs are kept as two 3-byte units)
                        if (v < 0x80) {
                            out += char(v);
                        } else if (v < 0x800) {
                            out += char(0xC0 | (v >> 6));
                            out += char(0x80 | (v & 0x3F));
                        } else {
                            out += char(0xE0 | (v >> 12));
                            out += char(0x80 | ((v >> 6) & 0x3F));
                            out += char(0x80 | (v & 0x3F));
                        }
                        break;
                    }
                    default: return fail("bad escape");
                }
            } else {
                out += c;
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool integer(int64_t &v) {
        ws();
        if (p >= end || *p < '0' || *p > '9') return fail("expected a non-negative integer");
        v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            if (v > (INT64_MAX - 9) / 10) return fail("integer too large");
            v = v * 10 + (*p++ - '0');
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return fail("expected an integer");
        return true;
    }
    bool skip(int depth = 0) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("truncated value");
        if (*p == '"') {
            std::string s;
            return string(s);
        }
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            ++p;
            if (eat(close)) return true;
            do {
                if (obj) {
                    std::string k;
                    if (!string(k) || !eat(':')) return fail("bad object");
                }
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(close) || fail("bad container");
        }
        // number, true, false, null
        const char *q = p;
        while (p < end && (std::strchr("+-.eE0123456789", *p) || (*p >= 'a' && *p <= 'z'))) ++p;
        return p > q || fail("unexpected character");
    }
};

struct DtypeName {
    const char *name;
    int32_t code;
    int size;
};
constexpr DtypeName kDtypes[] = {
    {"F32", DTTS_DT_F32, 4},   {"F16", DTTS_DT_F16, 2},    {"BF16", DTTS_DT_BF16, 2}, {"F64", DTTS_DT_F64, 8},
    {"I64", DTTS_DT_I64, 8},   {"I32", DTTS_DT_I32, 4},    {"I16", DTTS_DT_I16, 2},   {"I8", DTTS_DT_I8, 1},
    {"U8", DTTS_DT_U8, 1},     {"BOOL", DTTS_DT_BOOL, 1},  {"U16", DTTS_DT_OTHER, 2}, {"U32", DTTS_DT_OTHER, 4},
    {"U64", DTTS_DT_OTHER, 8}, {"F8_E4M3", DTTS_DT_OTHER, 1}, {"F8_E5M2", DTTS_DT_OTHER, 1},
};

bool parse_entry(Json &js, dtts_checkpoint::Entry &e, int &esize) {
    if (!js.eat('{')) return js.fail("expected an object for a tensor");
    bool have_dtype = false, have_shape = false, have_offsets = false;
    if (!js.eat('}')) {
        do {
            std::string key;
            if (!js.string(key) || !js.eat(':')) return js.fail("bad tensor entry");
            if (key == "dtype") {
                std::string d;
                if (!js.string(d)) return false;
                esize = 0;
                for (const DtypeName &n : kDtypes)
                    if (d == n.name) {
                        e.dtype = n.code;
                        esize = n.size;
                    }
                if (!esize) return js.fail("unknown dtype");
                have_dtype = true;
            } else if (key == "shape") {
                if (!js.eat('[')) return js.fail("shape is not an array");
                e.ndim = 0;
                if (!js.eat(']')) {
                    do {
                        int64_t v;
                        if (!js.integer(v)) return false;
                        if (e.ndim >= DTTS_TENSOR_MAX_DIMS) return js.fail("more than 8 dimensions");
                        e.shape[e.ndim++] = v;
                    } while (js.eat(','));
                    if (!js.eat(']')) return js.fail("bad shape");
                }
                have_shape = true;
            } else if (key == "data_offsets") {
                int64_t a, b;
                if (!js.eat('[') || !js.integer(a) || !js.eat(',') || !js.integer(b) || !js.eat(']'))
                    return js.fail("bad data_offsets");
                e.begin = static_cast<size_t>(a);
                e.end = static_cast<size_t>(b);
                have_offsets = true;
            } else if (!js.skip()) {
                return false;
            }
        } while (js.eat(','));
        if (!js.eat('}')) return js.fail("bad tensor entry");
    }
    if (!have_dtype || !have_shape || !have_offsets) return js.fail("a tensor entry lacks dtype, shape or data_offsets");
    return true;
}

int parse_header(dtts_checkpoint *ck, const char *hdr, size_t len, const char *path) {
    Json js{hdr, hdr + len, {}};
    const char *name = "dtts_checkpoint_open";
    DTTS_REQUIRE(js.eat('{'), "%s: %s: header is not a JSON object", name, path);
    if (!js.eat('}')) {
        do {
            std::string key;
            if (!js.string(key) || !js.eat(':')) {
                js.fail("bad header object");
                break;
            }
            if (key == "__metadata__") {
                if (!js.skip()) break;
                continue;
            }
            dtts_checkpoint::Entry e;
            e.name = key;
            int esize = 0;
            if (!parse_entry(js, e, esize)) break;
            // The element count is bounded so that numel * esize stays below 2^62 and cannot wrap
            // (a [2^61 + 1] F64 entry would wrap to 8 bytes); the byte count is compared after.
            bool empty = false;
            for (int i = 0; i < e.ndim; ++i) {
                DTTS_REQUIRE(e.shape[i] >= 0, "%s: %s: tensor %s: negative dimension", name, path, key.c_str());
                empty = empty || e.shape[i] == 0;
            }
            uint64_t numel = empty ? 0 : 1;
            const uint64_t most = (uint64_t(1) << 62) / uint64_t(esize);
            for (int i = 0; i < e.ndim && !empty; ++i) {
                DTTS_REQUIRE(numel <= most / uint64_t(e.shape[i]), "%s: %s: tensor %s: shape too large", name, path,
                             key.c_str());
                numel *= uint64_t(e.shape[i]);
            }
            DTTS_REQUIRE(e.begin <= e.end && e.end <= ck->data_size,
                         "%s: %s: tensor %s: data_offsets [%zu, %zu) outside the %zu-byte buffer", name, path,
                         key.c_str(), e.begin, e.end, ck->data_size);
            DTTS_REQUIRE(e.end - e.begin == numel * uint64_t(esize),
                         "%s: %s: tensor %s: %zu bytes for %llu elements of %d bytes", name, path, key.c_str(),
                         e.end - e.begin, (unsigned long long)numel, esize);
            DTTS_REQUIRE(ck->index.emplace(key, ck->entries.size()).second, "%s: %s: tensor %s listed twice", name,
                         path, key.c_str());
            ck->entries.push_back(std::move(e));
        } while (js.eat(','));
        if (js.err.empty() && !js.eat('}')) js.fail("bad header object");
    }
    DTTS_REQUIRE(js.err.empty(), "%s: %s: header: %s at byte %lld", name, path, js.err.c_str(),
                 (long long)(js.p - hdr));
    return DTTS_OK;
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ double load_f64(const void *src, int dtype, int64_t i) {
    switch (dtype) {
        case DTTS_DT_F32: return static_cast<const float *>(src)[i];
        case DTTS_DT_F16: return static_cast<float>(static_cast<const half_t *>(src)[i]);
        case DTTS_DT_BF16: return __uint_as_float(uint32_t(static_cast<const uint16_t *>(src)[i]) << 16);
        default: return static_cast<const double *>(src)[i];
    }
}

// Exactly representable in f32 for f32/f16/bf16 sources; an f64 source is rounded to f32 first
// (so every f16 result is one rounding of an f32 value, as a cast of the f32 tensor would be).
__device__ __forceinline__ float load_f32(const void *src, int dtype, int64_t i) {
    float f = static_cast<float>(load_f64(src, dtype, i));
    // keeps the f32 value: without it the compiler may fuse a following f32 -> f16 cast of an f64
    // source into one f64 -> f16 rounding, which differs where the two roundings do
    asm volatile("" : "+v"(f));
    return f;
}

__global__ __launch_bounds__(256) void cvt_f16_kernel(const void *src, int dtype, half_t *dst, int64_t n) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        dst[i] = static_cast<half_t>(load_f32(src, dtype, i));
}

__global__ __launch_bounds__(256) void cvt_f32_kernel(const void *src, int dtype, float *dst, int64_t n) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        dst[i] = load_f32(src, dtype, i);
}

__global__ __launch_bounds__(256) void cvt_f32_scaled_kernel(const void *src, int dtype, float *dst, int64_t n,
                                                              float scale) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        dst[i] = load_f32(src, dtype, i) * scale;
}

__global__ __launch_bounds__(256) void cvt_cols_kernel(const void *src, int dtype, half_t *dst, int64_t rows,
                                                        int64_t cols, int64_t ld, int64_t col0) {
    const int64_t n = rows * cols;
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
        const int64_t r = i / cols, c = i - r * cols;
        dst[r * ld + col0 + c] = static_cast<half_t>(load_f32(src, dtype, i));
    }
}

// [rows, cols] -> [cols, rows] through a 32 x 33 tile: reads along a source row, writes along a
// destination row.
__global__ __launch_bounds__(256) void cvt_transpose_kernel(const void *src, int dtype, half_t *dst, int64_t rows,
                                                             int64_t cols) {
    __shared__ float tile[32][33];
    const int64_t r0 = int64_t(blockIdx.y) * 32, c0 = int64_t(blockIdx.x) * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows of 32 per pass
    for (int j = ty; j < 32; j += 8) {
        const int64_t r = r0 + j, c = c0 + tx;
        tile[j][tx] = (r < rows && c < cols) ? load_f32(src, dtype, r * cols + c) : 0.0f;
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const int64_t c = c0 + j, r = r0 + tx;
        if (c < cols && r < rows) dst[c * rows + r] = static_cast<half_t>(tile[tx][j]);
    }
}

// dst[o, t*cin + i] = src[o, i, t]
__global__ __launch_bounds__(256) void cvt_tap_major_kernel(const void *src, int dtype, half_t *dst, int64_t cout,
                                                             int64_t cin, int64_t k) {
    const int64_t n = cout * k * cin;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) {
        const int64_t i = e % cin, t = (e / cin) % k, o = e / (cin * k);
        dst[e] = static_cast<half_t>(load_f32(src, dtype, (o * cin + i) * k + t));
    }
}

// dst[p*cout + co, t*cin + ci] = src[ci, co, (m-1-t)*stride + p], m = kernel / stride
__global__ __launch_bounds__(256) void cvt_transpose_tap_kernel(const void *src, int dtype, half_t *dst, int64_t cin,
                                                                 int64_t cout, int64_t kernel, int64_t stride) {
    const int64_t m = kernel / stride;
    const int64_t n = stride * cout * m * cin;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) {
        const int64_t ci = e % cin, t = (e / cin) % m, nn = e / (cin * m);
        const int64_t p = nn / cout, co = nn - p * cout;
        dst[e] = static_cast<half_t>(load_f32(src, dtype, (ci * cout + co) * kernel + (m - 1 - t) * stride + p));
    }
}

__global__ __launch_bounds__(256) void cvt_repeat_kernel(const void *src, int dtype, half_t *dst, int64_t n,
                                                          int64_t times) {
    const int64_t total = n * times;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256)
        dst[e] = static_cast<half_t>(load_f32(src, dtype, e % n));
}

// exp in f64, rounded once to f32: the correctly rounded f32 exp of the f32 parameter
__global__ __launch_bounds__(256) void snake_fold_kernel(const void *alog, const void *blog, int dtype, float *alpha,
                                                          float *brecip, int64_t n) {
#pragma clang fp contract(off)
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
        alpha[i] = static_cast<float>(exp(static_cast<double>(load_f32(alog, dtype, i))));
        const float eb = static_cast<float>(exp(static_cast<double>(load_f32(blog, dtype, i))));
        brecip[i] = 1.0f / (eb + 1e-9f);
    }
}

__global__ __launch_bounds__(256) void codebook_fold_kernel(const void *sum, const void *usage, int dtype, float eps,
                                                             float *dst, int64_t size, int64_t dim) {
    const int64_t n = size * dim;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) {
        const float u = load_f32(usage, dtype, e / dim);
        dst[e] = load_f32(sum, dtype, e) / fmaxf(u, eps);
    }
}

// Half a wave per 32-weight block: lane j holds weight j; amax over the 32 lanes by shuffles;
// d = amax / 127, id = 1/d (0 for an all-zero block), q = round-half-away(x * id).
__global__ __launch_bounds__(256) void q8_0_quantize_kernel(const void *w, int dtype, uint8_t *blocks,
                                                             int64_t nblocks) {
#pragma clang fp contract(off)
    const int j = threadIdx.x & 31;
    for (int64_t b = (blockIdx.x * int64_t(256) + threadIdx.x) >> 5; b < nblocks; b += (int64_t(gridDim.x) * 256) >> 5) {
        const float x = load_f32(w, dtype, b * 32 + j);
        float amax = fabsf(x);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *blk = blocks + b * 34;
        blk[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(roundf(x * id)));
        if (j == 0) {
            const half_t dh = static_cast<half_t>(d);
            uint16_t bits;
            __builtin_memcpy(&bits, &dh, 2);
            *reinterpret_cast<uint16_t *>(blk) = bits;
        }
    }
}

bool float_dtype(int32_t dtype) {
    return dtype == DTTS_DT_F32 || dtype == DTTS_DT_F16 || dtype == DTTS_DT_BF16 || dtype == DTTS_DT_F64;
}

int dtype_size(int32_t dtype) {
    return dtype == DTTS_DT_F64 ? 8 : dtype == DTTS_DT_F32 ? 4 : 2;
}

#define CVT_CHECK(name, src, dtype, dst)                                                                           \
    do {                                                                                                           \
        DTTS_REQUIRE(src && dst, "%s: null pointer", name);                                                        \
        DTTS_REQUIRE(::dtts::float_dtype(dtype), "%s: dtype %d is not a float type (F32, F16, BF16, F64)", name,  \
                     static_cast<int>(dtype));                                                                     \
        DTTS_REQUIRE(::dtts::aligned(src, ::dtts::dtype_size(dtype)), "%s: source misaligned for its dtype", name); \
    } while (0)

}  // namespace
}  // namespace dtts

// ---------------------------------------------------------------- reader entry points

extern "C" int dtts_checkpoint_open(const char *path, dtts_checkpoint **out) {
    const char *name = "dtts_checkpoint_open";
    DTTS_REQUIRE(path && out, "%s: null argument", name);
    *out = nullptr;
    dtts_checkpoint *ck = new (std::nothrow) dtts_checkpoint();
    DTTS_REQUIRE(ck, "%s: out of host memory", name);
    auto bail = [&](int rc) {
        dtts_checkpoint_close(ck);
        return rc;
    };
    ck->fd = ::open(path, O_RDONLY);
    if (ck->fd < 0) {
        dtts::set_error("%s: mapping %s: %s", name, path, std::strerror(errno));
        return bail(DTTS_ERR_INVALID);
    }
    struct stat st{};
    if (fstat(ck->fd, &st) != 0 || st.st_size < 8) {
        dtts::set_error("%s: %s: not a safetensors file (%lld bytes)", name, path, (long long)st.st_size);
        return bail(DTTS_ERR_INVALID);
    }
    ck->size = static_cast<size_t>(st.st_size);
    ck->map = mmap(nullptr, ck->size, PROT_READ, MAP_PRIVATE, ck->fd, 0);
    if (ck->map == MAP_FAILED) {
        ck->map = nullptr;
        dtts::set_error("%s: mapping %s: %s", name, path, std::strerror(errno));
        return bail(DTTS_ERR_INVALID);
    }
    const unsigned char *b = static_cast<const unsigned char *>(ck->map);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | b[i];
    if (hlen > ck->size - 8) {
        dtts::set_error("%s: %s: header length %llu exceeds the file (%zu bytes)", name, path, (unsigned long long)hlen,
                        ck->size);
        return bail(DTTS_ERR_INVALID);
    }
    ck->data = reinterpret_cast<const char *>(b) + 8 + hlen;
    ck->data_size = ck->size - 8 - static_cast<size_t>(hlen);
    const int rc = dtts::parse_header(ck, reinterpret_cast<const char *>(b) + 8, static_cast<size_t>(hlen), path);
    if (rc != DTTS_OK) return bail(rc);
    *out = ck;
    return DTTS_OK;
}

extern "C" void dtts_checkpoint_close(dtts_checkpoint *ck) {
    if (!ck) return;
    if (ck->map) munmap(ck->map, ck->size);
    if (ck->fd >= 0) ::close(ck->fd);
    delete ck;
}

extern "C" int64_t dtts_checkpoint_count(const dtts_checkpoint *ck) {
    return ck ? static_cast<int64_t>(ck->entries.size()) : 0;
}

namespace {
void fill_info(const dtts_checkpoint *ck, const dtts_checkpoint::Entry &e, dtts_tensor_info *out) {
    out->name = e.name.c_str();
    out->dtype = e.dtype;
    out->ndim = e.ndim;
    for (int i = 0; i < DTTS_TENSOR_MAX_DIMS; ++i) out->shape[i] = i < e.ndim ? e.shape[i] : 0;
    out->data = ck->data + e.begin;
    out->bytes = e.end - e.begin;
}
}  // namespace

extern "C" int dtts_checkpoint_at(const dtts_checkpoint *ck, int64_t index, dtts_tensor_info *out) {
    DTTS_REQUIRE(ck && out, "dtts_checkpoint_at: null argument");
    DTTS_REQUIRE(index >= 0 && index < static_cast<int64_t>(ck->entries.size()),
                 "dtts_checkpoint_at: index %lld outside [0, %zu)", (long long)index, ck->entries.size());
    fill_info(ck, ck->entries[static_cast<size_t>(index)], out);
    return DTTS_OK;
}

extern "C" int dtts_checkpoint_get(const dtts_checkpoint *ck, const char *name, dtts_tensor_info *out) {
    DTTS_REQUIRE(ck && name && out, "dtts_checkpoint_get: null argument");
    const auto it = ck->index.find(name);
    DTTS_REQUIRE(it != ck->index.end(), "missing tensor %s", name);
    fill_info(ck, ck->entries[it->second], out);
    return DTTS_OK;
}

// ---------------------------------------------------------------- conversion entry points

using dtts::grid_for;
using dtts::half_t;

extern "C" int dtts_convert_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t n, hipStream_t stream) {
    const char *name = "dtts_convert_f16";
    DTTS_REQUIRE(n >= 0, "%s: negative size", name);
    if (n == 0) return DTTS_OK;
    CVT_CHECK(name, src, dtype, dst);
    dtts::cvt_f16_kernel<<<grid_for(n, 256), 256, 0, stream>>>(src, dtype, reinterpret_cast<half_t *>(dst), n);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_f32(const void *src, int32_t dtype, float *dst, int64_t n, hipStream_t stream) {
    const char *name = "dtts_convert_f32";
    DTTS_REQUIRE(n >= 0, "%s: negative size", name);
    if (n == 0) return DTTS_OK;
    CVT_CHECK(name, src, dtype, dst);
    dtts::cvt_f32_kernel<<<grid_for(n, 256), 256, 0, stream>>>(src, dtype, dst, n);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_f32_scaled(const void *src, int32_t dtype, float *dst, int64_t n, float scale,
                                       hipStream_t stream) {
    const char *name = "dtts_convert_f32_scaled";
    DTTS_REQUIRE(n >= 0, "%s: negative size", name);
    if (n == 0) return DTTS_OK;
    CVT_CHECK(name, src, dtype, dst);
    dtts::cvt_f32_scaled_kernel<<<grid_for(n, 256), 256, 0, stream>>>(src, dtype, dst, n, scale);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_f16_cols(const void *src, int32_t dtype, dtts_f16 *dst, int64_t rows, int64_t cols,
                                     int64_t ld, int64_t col0, hipStream_t stream) {
    const char *name = "dtts_convert_f16_cols";
    DTTS_REQUIRE(rows >= 0 && cols >= 0 && col0 >= 0 && col0 + cols <= ld, "%s: columns [%lld, %lld) outside %lld",
                 name, (long long)col0, (long long)(col0 + cols), (long long)ld);
    if (rows == 0 || cols == 0) return DTTS_OK;
    CVT_CHECK(name, src, dtype, dst);
    dtts::cvt_cols_kernel<<<grid_for(rows * cols, 256), 256, 0, stream>>>(src, dtype, reinterpret_cast<half_t *>(dst),
                                                                          rows, cols, ld, col0);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_transpose_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t rows, int64_t cols,
                                          hipStream_t stream) {
    const char *name = "dtts_convert_transpose_f16";
    DTTS_REQUIRE(rows >= 0 && cols >= 0 && rows < (int64_t(1) << 36) && cols < (int64_t(1) << 36), "%s: bad shape",
                 name);
    if (rows == 0 || cols == 0) return DTTS_OK;
    CVT_CHECK(name, src, dtype, dst);
    DTTS_REQUIRE((cols + 31) / 32 < (int64_t(1) << 31) && (rows + 31) / 32 < 65536, "%s: shape too large", name);
    const dim3 grid(static_cast<unsigned>((cols + 31) / 32), static_cast<unsigned>((rows + 31) / 32));
    dtts::cvt_transpose_kernel<<<grid, 256, 0, stream>>>(src, dtype, reinterpret_cast<half_t *>(dst), rows, cols);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_tap_major_f16(const void *w_oik, int32_t dtype, dtts_f16 *dst, int64_t cout, int64_t cin,
                                          int64_t k, hipStream_t stream) {
    const char *name = "dtts_convert_tap_major_f16";
    DTTS_REQUIRE(cout > 0 && cin > 0 && k > 0, "%s: bad shape", name);
    CVT_CHECK(name, w_oik, dtype, dst);
    dtts::cvt_tap_major_kernel<<<grid_for(cout * cin * k, 256), 256, 0, stream>>>(
        w_oik, dtype, reinterpret_cast<half_t *>(dst), cout, cin, k);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_transpose_tap_major_f16(const void *w_iok, int32_t dtype, dtts_f16 *dst, int64_t cin,
                                                    int64_t cout, int64_t kernel, int64_t stride,
                                                    hipStream_t stream) {
    const char *name = "dtts_convert_transpose_tap_major_f16";
    DTTS_REQUIRE(cin > 0 && cout > 0 && kernel > 0 && stride > 0, "%s: bad shape", name);
    DTTS_REQUIRE(kernel % stride == 0, "%s: polyphase form needs kernel divisible by stride, got k=%lld stride=%lld",
                 name, (long long)kernel, (long long)stride);
    CVT_CHECK(name, w_iok, dtype, dst);
    dtts::cvt_transpose_tap_kernel<<<grid_for(cin * cout * kernel, 256), 256, 0, stream>>>(
        w_iok, dtype, reinterpret_cast<half_t *>(dst), cin, cout, kernel, stride);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_repeat_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t n, int64_t times,
                                       hipStream_t stream) {
    const char *name = "dtts_convert_repeat_f16";
    DTTS_REQUIRE(n > 0 && times > 0, "%s: bad shape", name);
    CVT_CHECK(name, src, dtype, dst);
    dtts::cvt_repeat_kernel<<<grid_for(n * times, 256), 256, 0, stream>>>(src, dtype, reinterpret_cast<half_t *>(dst),
                                                                          n, times);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_snake_fold(const void *alpha_log, const void *beta_log, int32_t dtype, float *alpha,
                                       float *brecip, int64_t n, hipStream_t stream) {
    const char *name = "dtts_convert_snake_fold";
    DTTS_REQUIRE(n > 0, "%s: bad size", name);
    CVT_CHECK(name, alpha_log, dtype, alpha);
    CVT_CHECK(name, beta_log, dtype, brecip);
    dtts::snake_fold_kernel<<<grid_for(n, 256), 256, 0, stream>>>(alpha_log, beta_log, dtype, alpha, brecip, n);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_codebook_fold(const void *embedding_sum, const void *cluster_usage, int32_t dtype,
                                          float eps, float *dst, int64_t size, int64_t dim, hipStream_t stream) {
    const char *name = "dtts_convert_codebook_fold";
    DTTS_REQUIRE(size > 0 && dim > 0, "%s: bad shape", name);
    CVT_CHECK(name, embedding_sum, dtype, dst);
    CVT_CHECK(name, cluster_usage, dtype, dst);
    dtts::codebook_fold_kernel<<<grid_for(size * dim, 256), 256, 0, stream>>>(embedding_sum, cluster_usage, dtype, eps,
                                                                              dst, size, dim);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_convert_q8_0(const void *w, int32_t dtype, void *blocks, int64_t rows, int64_t k,
                                 hipStream_t stream) {
    const char *name = "dtts_convert_q8_0";
    DTTS_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "%s: k = %lld is not a multiple of 32", name, (long long)k);
    if (rows == 0) return DTTS_OK;
    CVT_CHECK(name, w, dtype, blocks);
    DTTS_REQUIRE(dtts::aligned(blocks, 2), "%s: blocks must be 2-byte aligned", name);
    const int64_t nb = rows * (k / 32);
    dtts::q8_0_quantize_kernel<<<grid_for(nb * 32, 256), 256, 0, stream>>>(w, dtype, static_cast<uint8_t *>(blocks),
                                                                           nb);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}
