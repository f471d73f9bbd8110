// The two-pass weight loader shared by the model loaders: a plan written once runs first as a
// dry pass (tensor lookups, dtype and shape checks, the arena's size) and then for real
// (each raw tensor uploaded once into a device copy of the file's byte buffer, converted into
// the arena by the dtts_convert_* kernels).
#pragma once

#include <string>
#include <unordered_set>

#include "common.hpp"

namespace dtts {
namespace {

inline size_t round256(size_t v) { return (v + 255) & ~size_t(255); }

struct Build {
    const char *who = "loader";  // the entry point, for messages
    const dtts_checkpoint *ck = nullptr;
    hipStream_t stream = nullptr;
    bool dry = true;
    char *arena = nullptr;       // second pass: the weights
    char *raw = nullptr;         // second pass: device copy of the file's byte buffer
    const char *host0 = nullptr; // first byte of the file's byte buffer (host mapping)
    size_t used = 0;
    char *q8tmp = nullptr;            // second pass: GGML blocks of one projection before its repack
    size_t q8max = 0;                 // first pass: the largest such staging
    std::unordered_set<size_t> sent;  // byte offsets of the raw tensors uploaded
    int rc = DTTS_OK;

    bool fail(int code) {
        if (rc == DTTS_OK) rc = code;
        return false;
    }
    bool ok(int code) { return code == DTTS_OK || fail(code); }

    // The tensor `name` of a float dtype, with exactly `shape` (when `shape` is empty: any shape
    // of `numel` elements).
    bool need(const std::string &name, std::initializer_list<int64_t> shape, dtts_tensor_info &t,
              int64_t numel = 0) {
        if (rc != DTTS_OK) return false;
        if (dtts_checkpoint_get(ck, name.c_str(), &t) != DTTS_OK) return fail(DTTS_ERR_INVALID);
        if (t.dtype != DTTS_DT_F32 && t.dtype != DTTS_DT_F16 && t.dtype != DTTS_DT_BF16 && t.dtype != DTTS_DT_F64) {
            set_error("%s: %s: dtype %d is not a float type", who, name.c_str(), t.dtype);
            return fail(DTTS_ERR_INVALID);
        }
        bool match;
        if (shape.size() == 0) {
            int64_t n = 1;
            for (int i = 0; i < t.ndim; ++i) n *= t.shape[i];
            match = n == numel;
        } else {
            match = static_cast<int>(shape.size()) == t.ndim;
            int i = 0;
            for (int64_t d : shape) match = match && t.shape[i++] == d;
        }
        if (!match) {
            std::string got, want;
            for (int i = 0; i < t.ndim; ++i) got += (i ? ", " : "") + std::to_string(t.shape[i]);
            if (shape.size() == 0) {
                want = std::to_string(numel) + " elements";
            } else {
                int i = 0;
                for (int64_t d : shape) want += (i++ ? ", " : "") + std::to_string(d);
                want = "[" + want + "]";
            }
            set_error("%s: %s: shape [%s], expected %s", who, name.c_str(), got.c_str(), want.c_str());
            return fail(DTTS_ERR_INVALID);
        }
        return true;
    }

    // The raw tensor on the device, uploaded on first use (second pass only).
    const void *src(const dtts_tensor_info &t) {
        const size_t off = static_cast<size_t>(static_cast<const char *>(t.data) - host0);
        if (sent.insert(off).second && t.bytes) {
            const hipError_t e = hipMemcpyAsync(raw + off, t.data, t.bytes, hipMemcpyHostToDevice, stream);
            if (e != hipSuccess) {
                set_error("%s: uploading %s: %s", who, t.name, hipGetErrorString(e));
                fail(DTTS_ERR_HIP);
            }
        }
        return raw + off;
    }

    template <typename T>
    T *alloc(int64_t n) {
        const size_t at = used;
        used += round256(sizeof(T) * static_cast<size_t>(n));
        return dry ? nullptr : reinterpret_cast<T *>(arena + at);
    }

    // --- the conversions the plan uses; each returns the arena pointer (nullptr on the first pass)
    dtts_f16 *f16(const dtts_tensor_info &t, int64_t n) {
        dtts_f16 *d = alloc<dtts_f16>(n);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16(src(t), t.dtype, d, n, stream));
        return d;
    }
    float *f32(const dtts_tensor_info &t, int64_t n) {
        float *d = alloc<float>(n);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f32(src(t), t.dtype, d, n, stream));
        return d;
    }
    dtts_f16 *tap(const dtts_tensor_info &t, int64_t cout, int64_t cin, int64_t k) {
        dtts_f16 *d = alloc<dtts_f16>(cout * cin * k);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_tap_major_f16(src(t), t.dtype, d, cout, cin, k, stream));
        return d;
    }
    dtts_f16 *ttap(const dtts_tensor_info &t, int64_t cin, int64_t cout, int64_t kernel, int64_t stride) {
        dtts_f16 *d = alloc<dtts_f16>(cin * cout * kernel);
        if (!dry && rc == DTTS_OK)
            ok(dtts_convert_transpose_tap_major_f16(src(t), t.dtype, d, cin, cout, kernel, stride, stream));
        return d;
    }
    dtts_f16 *repeat(const dtts_tensor_info &t, int64_t n, int64_t times) {
        dtts_f16 *d = alloc<dtts_f16>(n * times);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_repeat_f16(src(t), t.dtype, d, n, times, stream));
        return d;
    }
    // rows of `t` ([rows, cols]) into rows [row0, row0 + rows) of `d` ([*, cols])
    void rows_into(const dtts_tensor_info &t, dtts_f16 *d, int64_t row0, int64_t rows, int64_t cols) {
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16(src(t), t.dtype, d + row0 * cols, rows * cols, stream));
    }
    void cols_into(const dtts_tensor_info &t, dtts_f16 *d, int64_t rows, int64_t cols, int64_t ld, int64_t col0) {
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16_cols(src(t), t.dtype, d, rows, cols, ld, col0, stream));
    }
    float *f32_scaled(const dtts_tensor_info &t, int64_t n, float scale) {
        float *d = alloc<float>(n);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f32_scaled(src(t), t.dtype, d, n, scale, stream));
        return d;
    }
    // both passes, after a plan: the raw staging covers the file's byte buffer from its first tensor
    static size_t raw_span(const dtts_checkpoint *ck, const char *&host0) {
        dtts_tensor_info t{};
        size_t span = 0;
        host0 = nullptr;
        for (int64_t i = 0; i < dtts_checkpoint_count(ck); ++i)
            if (dtts_checkpoint_at(ck, i, &t) == DTTS_OK && (!host0 || static_cast<const char *>(t.data) < host0))
                host0 = static_cast<const char *>(t.data);
        for (int64_t i = 0; i < dtts_checkpoint_count(ck); ++i)
            if (dtts_checkpoint_at(ck, i, &t) == DTTS_OK) {
                const size_t end = static_cast<size_t>(static_cast<const char *>(t.data) - host0) + t.bytes;
                if (end > span) span = end;
            }
        return span;
    }
    void snake(const std::string &prefix, int64_t c, const float *&alpha, const float *&brecip) {
        dtts_tensor_info a, b;
        if (!need(prefix + ".alpha", {}, a, c) || !need(prefix + ".beta", {}, b, c)) return;
        if (a.dtype != b.dtype) {
            set_error("%s: %s.alpha and .beta differ in dtype", who, prefix.c_str());
            fail(DTTS_ERR_INVALID);
            return;
        }
        float *pa = alloc<float>(c), *pb = alloc<float>(c);
        if (!dry && rc == DTTS_OK) {
            const void *sa = src(a), *sb = src(b);
            ok(dtts_convert_snake_fold(sa, sb, a.dtype, pa, pb, c, stream));
        }
        alpha = pa;
        brecip = pb;
    }
};

}  // namespace
}  // namespace dtts
