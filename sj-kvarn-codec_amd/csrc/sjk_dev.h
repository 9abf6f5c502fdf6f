// sjk_dev.h - device-side numeric primitives and format helpers shared by the HIP kernels.
//
// Numeric contract (the record bytes depend on it; reference sj_kvarn.h:647-731 and README.md:287-298):
//   * every + - * / rounds once: the library is compiled with -ffp-contract=off, so no FMA contraction;
//   * fp32 division and sqrtf are correctly rounded (hipcc default), denormals are kept;
//   * min/max are the ternary forms b<a?b:a and a<b?b:a (signed zero and NaN behaviour);
//   * float -> half rounds to nearest even (v_cvt_f16_f32, fp16 denormals kept) with NaN -> sign|0x7E00.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sjk.h"
#include "../../include/sjk_tables.h"

#define SJK_DEV static __device__ __forceinline__

namespace sjk {

// ---- format tables in constant memory (sj_kvarn.h:479-623), one copy per translation unit ----
static __constant__ uint16_t c_cb3k[512] = SJK_CB3_K_INIT;
static __constant__ uint16_t c_cb3v[512] = SJK_CB3_V_INIT;
static __constant__ uint16_t c_cb2k[256] = SJK_CB2_K_INIT;
static __constant__ uint16_t c_cb2v[256] = SJK_CB2_V_INIT;
static __constant__ uint32_t c_tq6_cent_bits[64] = SJK_TQ6_CENTROID_BITS_INIT;
static __constant__ uint32_t c_tq6_mid_bits[63] = SJK_TQ6_MIDPOINT_BITS_INIT;

SJK_DEV float bits_f(uint32_t w) { return __uint_as_float(w); }
SJK_DEV float tq6_cent(int i) { return __uint_as_float(c_tq6_cent_bits[i]); }
SJK_DEV float tq6_mid(int i) { return __uint_as_float(c_tq6_mid_bits[i]); }
SJK_DEV uint32_t f_bits(float f) { return __float_as_uint(f); }

SJK_DEV float tmin(float a, float b) { return b < a ? b : a; }
SJK_DEV float tmax(float a, float b) { return a < b ? b : a; }
SJK_DEV double tmin(double a, double b) { return b < a ? b : a; }
SJK_DEV double tmax(double a, double b) { return a < b ? b : a; }

// float -> half as the reference rounds (sj_kvarn.h:693-711): IEEE round to nearest even with fp16 subnormals and
// overflow to +-inf, NaN -> sign | 0x7E00. v_cvt_f16_f32 is exactly that rounding under the kernels' default mode
// (round to nearest even, fp16 denormals kept); only a NaN needs the reference's canonical pattern. Checked on the
// device over all 2^32 float bit patterns, against numpy's cast as well (tests/test_gpu_full.py).
SJK_DEV uint16_t f32_to_f16(float f) {
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16) f);
    return f != f ? (uint16_t) (((f_bits(f) >> 16) & 0x8000u) | 0x7E00u) : h;
}

// half -> float, exact, signalling NaNs kept as they are (sj_kvarn.h:713-731)
SJK_DEV float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 31u) return bits_f(sign | 0x7F800000u | (m << 13));
    if (e != 0u) return bits_f(sign | ((e + 112u) << 23) | (m << 13));
    const float v = (float) m * 0x1p-24f;
    return sign ? -v : v;
}

// half -> float on the hardware converter: exact for every half except that it quiets signalling
// NaNs; used where only values matter (attention), never for bytes that are compared
SJK_DEV float f16_to_f32_fast(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

// ---- the host's NaN rule, for the paths that see non-finite values ----
// A stored NaN half keeps only its sign (sign | 0x7E00), so the sign of every NaN the arithmetic makes is part
// of the bytes. IEEE 754 leaves it unspecified; the reference's host build (x86-64 SSE) returns a quieted copy of
// its first NaN operand, and for an invalid operation with no NaN operand (inf - inf, 0 * inf) the default NaN,
// whose sign bit is set. gfx950 makes a positive NaN there. The x* operations below give the host's result from
// the hardware's: the kernels use them on a side / row / block that holds an infinity or a NaN (a per-wave or
// per-workgroup vote), so finite inputs keep the plain arithmetic. Where NaNs of both signs meet, the host's
// result is whichever operand its compiler placed first; these take the left one as written.
SJK_DEV float nan_of(float a) { return bits_f((f_bits(a) & 0x80000000u) | 0x7FC00000u); }
SJK_DEV double nan_of(double a) {
    return __longlong_as_double((long long) (((uint64_t) __double_as_longlong(a) & 0x8000000000000000ull) |
                                             0x7FF8000000000000ull));
}
SJK_DEV float x86_res(float r, float a, float b) {
    return a != a ? nan_of(a) : b != b ? nan_of(b) : r != r ? bits_f(0xFFC00000u) : r;
}
SJK_DEV double x86_res(double r, double a, double b) {
    return a != a ? nan_of(a) : b != b ? nan_of(b) : r != r ? __longlong_as_double((long long) 0xFFF8000000000000ull) : r;
}
SJK_DEV float xadd(float a, float b) { return x86_res(a + b, a, b); }
SJK_DEV float xsub(float a, float b) { return x86_res(a - b, a, b); }
SJK_DEV float xmul(float a, float b) { return x86_res(a * b, a, b); }
SJK_DEV float xdiv(float a, float b) { return x86_res(a / b, a, b); }
SJK_DEV double xadd(double a, double b) { return x86_res(a + b, a, b); }
SJK_DEV double xsub(double a, double b) { return x86_res(a - b, a, b); }
// conversions keep a NaN's sign (cvtss2sd / cvtsd2ss)
SJK_DEV double f2d_x(float a) {
    return a != a ? __longlong_as_double((long long) (((uint64_t) (f_bits(a) & 0x80000000u) << 32) | 0x7FF8000000000000ull))
                  : (double) a;
}
SJK_DEV float d2f_x(double a) {
    return a != a ? bits_f(((uint32_t) (((uint64_t) __double_as_longlong(a)) >> 32) & 0x80000000u) | 0x7FC00000u)
                  : (float) a;
}
// a half that is an infinity or a NaN
SJK_DEV bool f16_nonfinite(uint16_t h) { return (h & 0x7C00u) == 0x7C00u; }

// one decoded value (sj_kvarn.h:1187-1207): ((q * scale) + zero) * column scale, with the host's NaN rule (a NaN
// scale half gives a NaN of its own sign)
SJK_DEV float dequant_x(float q, float scale, float zero, float col) { return xmul(xadd(xmul(q, scale), zero), col); }

// Correctly rounded float a / b from the double reciprocal yd = RN64(1/b): RN32(RN64(a * yd)), three VALU
// operations (two conversions and a double multiply). Why this is RN32(a / b) for float a, b > 0 whose
// quotient is a normal float:
//  * a / b is never a float midpoint: a midpoint m has an odd 25-bit significand M, and a = m * b would give a
//    the odd factor M * (odd part of b's significand), 25 significant bits or more;
//  * a / b lies at least 2^-49 |a / b| from every midpoint m: a - m*b is a nonzero multiple of
//    2^min(exp(a), exp(m) + exp(b)) (integer significands A < 2^24, M < 2^25, B < 2^24), so |a/b - m| >=
//    2^exp(m) / B >= 2^-49 m, or >= |a| / (A b) >= 2^-24 |a/b| when the exponent of a is the smaller;
//  * RN64(a * yd) = (a / b)(1 + d1)(1 + d2), |d1|, |d2| <= 2^-53, so it is within 2^-52 |a / b| of a / b, on
//    the same side of every midpoint, and RN32 of it is RN32(a / b) (an exact float quotient stays itself).
// The balance loop divides |a| <= 65504 (fp16 inputs and their quotients) by b in [exp(-0.3), exp(10)], so
// every quotient is at least 2^-54 and normal. +-0, +-inf and NaN numerators give the IEEE quotient too (the
// sign of a with b > 0; NaN stays NaN).
SJK_DEV float div_by_drecip(float a, double yd) { return (float) ((double) a * yd); }

// ---- record layout (sj_kvarn.h:761-900) ----
SJK_DEV bool frag_side(const sj_kvarn_layout & l, int bits) {
    return l.body == SJKVARN_BODY_SCALAR && bits == 4 && (l.D % 16) == 0 && (l.G % 16) == 0;
}

SJK_DEV int k_ch_idx(const sj_kvarn_layout & l, int d) {
    if (!frag_side(l, l.bits_k)) return d;
    const int c = d >> 4, dd = d & 15, jj = dd >> 1;
    return (jj & 3) * (l.D / 4) + c * 4 + (jj >> 2) * 2 + (dd & 1);
}

SJK_DEV int v_ch_idx(const sj_kvarn_layout & l, int d) {
    if (!frag_side(l, l.bits_v)) return d;
    return (d & 7) * (l.D / 8) + (d >> 4) * 2 + ((d >> 3) & 1);
}

SJK_DEV uint32_t code_bit(const sj_kvarn_layout & l, int t, int d, int is_v) {
    const int bits = is_v ? l.bits_v : l.bits_k;
    if (l.body == SJKVARN_BODY_TRELLIS) return ((uint32_t) d * (uint32_t) l.G + (uint32_t) t) * (uint32_t) bits;
    if (!frag_side(l, bits)) return ((uint32_t) t * (uint32_t) l.D + (uint32_t) d) * (uint32_t) bits;
    const int a = is_v ? d : t, b = is_v ? t : d;
    const int aa = a & 15, bb = b & 15;
    const uint32_t tile = (uint32_t) ((t >> 4) * (l.D / 16) + (d >> 4));
    const uint32_t word = tile * 32u + (uint32_t) (4 * (aa & 7) + ((bb >> 1) & 3));
    const uint32_t nib = (uint32_t) ((aa >> 3) + 2 * (bb >> 3) + 4 * (bb & 1));
    return word * 32u + nib * 4u;
}

SJK_DEV uint32_t get_code(const uint8_t * p, uint32_t bit, int bits) {
    const uint32_t sh = bit & 7u;
    uint32_t w = p[bit >> 3];
    if (sh + (uint32_t) bits > 8u) w |= (uint32_t) p[(bit >> 3) + 1] << 8;
    return (w >> sh) & ((1u << bits) - 1u);
}

SJK_DEV const uint16_t * codebook(int bits, int is_v) {
    if (bits == 3) return is_v ? c_cb3v : c_cb3k;
    return is_v ? c_cb2v : c_cb2k;
}

// trellis window of the code at (channel seq, token i): code << 6 | the 6 stream bits before it,
// zeros before the channel start (sj_kvarn.h:882-900)
SJK_DEV uint32_t trellis_window(const uint8_t * payload, int bits, int seq, int i) {
    const uint32_t bit = ((uint32_t) seq * SJKVARN_TRELLIS_SEQ + (uint32_t) i) * (uint32_t) bits;
    uint32_t w = get_code(payload, bit, bits) << SJKVARN_TRELLIS_HIST_BITS;
    for (int k = 1; k * bits < SJKVARN_TRELLIS_HIST_BITS + bits && k <= i; ++k) {
        const int sh = SJKVARN_TRELLIS_HIST_BITS - k * bits;
        const uint32_t c = get_code(payload, bit - (uint32_t) (k * bits), bits);
        w |= sh >= 0 ? (c << sh) : (c >> (-sh));
    }
    return w;
}

SJK_DEV float get_half(const uint8_t * rec, uint32_t off) {
    return f16_to_f32((uint16_t) (rec[off] | (rec[off + 1] << 8)));
}

// tq6_0 level: count of midpoints m with !(v < mid[m]), the result of the reference's 6-step binary
// search over the sorted midpoints (sj_kvarn.h:1211-1219); NaN -> 63. mid[] is an LDS or constant copy.
SJK_DEV int tq6_level(float v, const float * mid) {
    int idx = 0;
#pragma unroll
    for (int step = 32; step >= 1; step >>= 1) idx += (v < mid[idx + step - 1]) ? 0 : step;
    return idx;
}

// One run of a gather / scatter between device regions (sjk_copy_runs, sjk_rows.hip): bytes from src to dst.
struct CopyRun {
    uint64_t src, dst, bytes;
};

// Copy every run of the device table d_runs[n] (one launch; runs are copied with 16-byte accesses where src,
// dst and bytes allow it). 0 or SJK_ERR_DEVICE.
int sjk_copy_runs(const CopyRun * d_runs, int n, hipStream_t stream);

// Zero the dst range of every run of d_runs[n] (src unused), one launch. 0 or SJK_ERR_DEVICE.
int sjk_zero_runs(const CopyRun * d_runs, int n, hipStream_t stream);

// Copy n words from host memory to d_dst on `stream` through kernel arguments (one launch per WORD_BATCH words):
// nothing is read from host memory after the call returns. 0 or SJK_ERR_DEVICE.
constexpr uint32_t WORD_BATCH = 960;
struct WordBatch {
    uint32_t n;
    uint32_t v[WORD_BATCH];
};
int sjk_set_words(uint32_t * d_dst, const uint32_t * host, uint32_t n, hipStream_t stream);

// ---- attention workspace of a view (sjk_hip_view.work) ----
// [plan of a 4/4 sjk_hip_attend_dyn launch (its job table): WS_PLAN_BYTES] [staging of the host-array layer calls:
// ws_stage_bytes] [partial results: slots of 16 query rows x (m, l, O[D]) floats]
constexpr size_t WS_PLAN_BYTES = 4096;
inline size_t ws_stage_bytes(int D, int H) { return ((size_t) H * (size_t) D * 8u + 255u) & ~(size_t) 255u; }
__host__ __device__ inline size_t ws_slot_floats(int D) { return (size_t) 16 * (size_t) (D + 2); }
inline void * ws_plan(const sjk_hip_view & v) { return v.work; }
inline uint8_t * ws_stage(const sjk_hip_view & v) { return (uint8_t *) v.work + WS_PLAN_BYTES; }
inline float * ws_part(const sjk_hip_view & v) {
    return (float *) ((uint8_t *) v.work + WS_PLAN_BYTES + ws_stage_bytes(v.lay.D, v.n_head_kv));
}
// partial slots the view's workspace holds (0 without one)
inline size_t ws_part_slots(const sjk_hip_view & v) {
    const size_t head = WS_PLAN_BYTES + ws_stage_bytes(v.lay.D, v.n_head_kv);
    if (!v.work || v.work_bytes <= head || v.lay.D <= 0) return 0;
    return (v.work_bytes - head) / (ws_slot_floats(v.lay.D) * sizeof(float));
}
// the text sjk_last_error() returns on the calling thread (sjk_host.cpp)
void set_error(const char * what);

// partial slots that sjk_hip_workspace_bytes provides: every attention launch fits (sjk_attend3.hip)
int ws_slots(int n_head_kv);
// compute units of the current device
int n_cus();

}  // namespace sjk

#define SJK_CHECK_LAUNCH() (hipPeekAtLastError() == hipSuccess ? 0 : SJK_ERR_DEVICE)
