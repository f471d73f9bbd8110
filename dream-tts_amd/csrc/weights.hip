// Load-time weight layouts (host code): the permutations that turn checkpoint tensors into the
// operand layouts the kernels read. Pure index arithmetic, any element size.
#include <cstring>

#include "common.hpp"

namespace dtts {
namespace {

bool elem_ok(int64_t es) { return es == 1 || es == 2 || es == 4 || es == 8; }

inline void copy_elem(char *dst, const char *src, int64_t es) { std::memcpy(dst, src, static_cast<size_t>(es)); }

}  // namespace
}  // namespace dtts

using dtts::copy_elem;
using dtts::elem_ok;

extern "C" int dtts_tap_major_weight(const void *w_oik, void *w_tm, int64_t cout, int64_t cin, int64_t k,
                                     int64_t es) {
    DTTS_REQUIRE(w_oik && w_tm && cout > 0 && cin > 0 && k > 0 && elem_ok(es),
                 "dtts_tap_major_weight: bad arguments");
    const char *s = static_cast<const char *>(w_oik);
    char *d = static_cast<char *>(w_tm);
    for (int64_t o = 0; o < cout; ++o)
        for (int64_t i = 0; i < cin; ++i)
            for (int64_t t = 0; t < k; ++t)
                copy_elem(d + ((o * k + t) * cin + i) * es, s + ((o * cin + i) * k + t) * es, es);
    return DTTS_OK;
}

extern "C" int dtts_tap_weight_to_tap_major(const void *w_kio, void *w_tm, int64_t k, int64_t cin, int64_t cout,
                                            int64_t es) {
    DTTS_REQUIRE(w_kio && w_tm && cout > 0 && cin > 0 && k > 0 && elem_ok(es),
                 "dtts_tap_weight_to_tap_major: bad arguments");
    const char *s = static_cast<const char *>(w_kio);
    char *d = static_cast<char *>(w_tm);
    for (int64_t t = 0; t < k; ++t)
        for (int64_t i = 0; i < cin; ++i)
            for (int64_t o = 0; o < cout; ++o)
                copy_elem(d + ((o * k + t) * cin + i) * es, s + ((t * cin + i) * cout + o) * es, es);
    return DTTS_OK;
}

// Output column nn = p*cout + co (phase p of channel co); tap t of the causal form is tap group
// i = m-1-t of the transposed conv: w_tm[nn, t*cin + ci] = w[ci, co, i*stride + p].
extern "C" int dtts_transpose_tap_major_weight(const void *w_iok, void *w_tm, int64_t cin, int64_t cout,
                                               int64_t kernel, int64_t stride, int64_t es) {
    DTTS_REQUIRE(w_iok && w_tm && cin > 0 && cout > 0 && kernel > 0 && stride > 0 && elem_ok(es),
                 "dtts_transpose_tap_major_weight: bad arguments");
    DTTS_REQUIRE(kernel % stride == 0,
                 "dtts_transpose_tap_major_weight: polyphase form needs kernel divisible by stride, got k=%lld stride=%lld",
                 (long long)kernel, (long long)stride);
    const int64_t m = kernel / stride;
    const char *s = static_cast<const char *>(w_iok);
    char *d = static_cast<char *>(w_tm);
    for (int64_t p = 0; p < stride; ++p)
        for (int64_t co = 0; co < cout; ++co) {
            const int64_t nn = p * cout + co;
            for (int64_t t = 0; t < m; ++t) {
                const int64_t i = m - 1 - t;
                for (int64_t ci = 0; ci < cin; ++ci)
                    copy_elem(d + ((nn * m + t) * cin + ci) * es, s + ((ci * cout + co) * kernel + i * stride + p) * es, es);
            }
        }
    return DTTS_OK;
}

extern "C" int dtts_transpose_bias(const void *b, void *out, int64_t cout, int64_t stride, int64_t es) {
    DTTS_REQUIRE(b && out && cout > 0 && stride > 0 && elem_ok(es), "dtts_transpose_bias: bad arguments");
    const char *s = static_cast<const char *>(b);
    char *d = static_cast<char *>(out);
    for (int64_t p = 0; p < stride; ++p) std::memcpy(d + p * cout * es, s, static_cast<size_t>(cout * es));
    return DTTS_OK;
}
