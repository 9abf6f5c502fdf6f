// sjk_seal.hip - the seal (encode) kernel: fp16 rows or staging-ring rows -> sealed records.
//
// One workgroup of 1024 threads seals one SIDE (K or V) of one record (one group of G = 128 tokens of
// one KV head); grid = (records, 2). The two sides write disjoint byte ranges of the record, so no
// zeroing pass is needed: every byte of the record is written exactly once (or twice by the same
// thread for trellis scale/zero, refit last).
//
// Per side, with the tile [R][C] (K: rows = channels, cols = tokens; V: rows = tokens, cols = channels;
// reference sj_kvarn.h:1149-1174):
//   * the fp16 tile M lives in LDS ([R][C+2] halves: odd word stride, so column walks and row walks
//     by consecutive lanes are both bank-conflict free);
//   * balance (sj_kvarn.h:992-1012): 2*iters passes. Each pass recomputes cur = (M / s_col) / s_row on
//     the fly (the reference's `recompute`, fused into its consumer), sums the 8 contiguous chunks of
//     every column (or row) sequentially in double, combines them in the fixed tree order, takes the
//     m2 chunks with fma, and updates the log-domain scale of that column (row). The two divisions use
//     the scales' double reciprocals, one double product rounded to float, which is the correctly
//     rounded quotient here (sjk_dev.h div_by_drecip), so cur is bit-identical to the reference's;
//   * quantize (sj_kvarn.h:1112-1147): row min/max (ordered chunk combine, NaN-exact), then one thread
//     per 8 codes writes b bytes of payload (4-bit fragment order, token-major or channel-major);
//   * trellis (sj_kvarn.h:1025-1109): one wavefront per channel runs the 64-state Viterbi with one
//     state per lane (path metrics exchanged with ds_bpermute, branch choices packed in registers,
//     traceback with readlane), then one thread per row does the moment-matching refit.
#include "sjk_dev.h"

namespace sjk {

constexpr int SEAL_NT = 1024;
constexpr int SEAL_MAX_LAYERS = 64;

struct SealLayer {
    const uint8_t * ring;
    uint8_t * body;
    const uint32_t * blocks;
};

struct SealArgs {
    sj_kvarn_layout lay;
    int iters;
    int mode;        // 0: fp16 rows (k, v, row_stride); 1: staging ring of layers[]
    int H;
    int n_groups;    // groups per layer in this launch
    int n_layers;
    // mode 0
    const uint16_t * k;
    const uint16_t * v;
    size_t row_stride;
    uint8_t * body;
    // mode 1
    int staging;
    uint32_t S, cap, B_from;
    size_t stage_bytes;
    const int32_t * desc;    // sjk_hip_commit_dyn: [desc[B_OLD], desc[B]) replaces [B_from, B_from + n_groups G)
    SealLayer layers[SEAL_MAX_LAYERS];
};

// LDS image of one side (sized for D = 256, G = 128; D = 128 uses a prefix)
struct SealLds {
    uint16_t M[256 * 130];                 // [R][C+2] fp16 bits
    union {
        struct { double a[8 * 256], b[8 * 256]; } part;   // chunk partials (balance)
        struct { float lo[8 * 256], hi[8 * 256]; } mm;    // chunk min/max (quantize)
        uint8_t codes[256 * 128];                         // trellis codes [channel][token]
    } u;
    float srow[256], scol[256];
    double yrow[256], ycol[256];            // RN64(1 / scale)
    double lrow[256], lcol[256];
    float qlo[256], qstep[256];
    float cbf[512];
    float tq6c[64];
};

// ------------------------------------------------------------------------------------------------
// loading the side's tile into LDS
// ------------------------------------------------------------------------------------------------

// The side's tile: fp16 rows (mode 0) or the staging ring rows of [B_from + g G, + G) (mode 1), tq6_0 dequantized
// and rounded to half as layer_seal stages them (sj_kvarn.h:1502-1509: cent[code] * f16->f32(norm), then RNE to
// half) or F16 staging as stored. Thread unit: 8 consecutive values of one token row (one slot computation and
// four 16-bit loads of the tq6_0 block for the 8 codes; blocks are 98 bytes, so 2-byte aligned).
// Returns nonzero when this thread loaded an infinity or a NaN (bit 15 of the OR of |h| + 0x400).
template <int R, int C, bool IS_V>
SJK_DEV uint32_t load_tile(const SealArgs & a, int il, int g, int h, uint32_t B_from, SealLds & s) {
    constexpr int D = IS_V ? C : R, G = IS_V ? R : C, CP = C + 2, U = D / 8;
    static_assert(D % 128 == 0, "whole tq6_0 blocks per row");
    const int tid = threadIdx.x;
    uint32_t nf = 0;
    for (int u = tid; u < G * U; u += SEAL_NT) {
        const int t = u / U, d0 = 8 * (u % U);
        uint16_t hv[8];
        if (a.mode == 0) {
            const uint16_t * src = (IS_V ? a.v : a.k) + (size_t) (g * G + t) * a.row_stride + (size_t) h * D + d0;
#pragma unroll
            for (int k = 0; k < 8; ++k) hv[k] = src[k];
        } else {
            const uint32_t pos = B_from + (uint32_t) (g * G + t);
            const uint32_t slot = (pos - a.S) % a.cap;
            const uint8_t * row = a.layers[il].ring + ((size_t) slot * a.H + h) * 2 * a.stage_bytes +
                                  (IS_V ? a.stage_bytes : 0);
            if (a.staging == SJKVARN_STAGING_F16) {
                const uint16_t * p = (const uint16_t *) row + d0;
#pragma unroll
                for (int k = 0; k < 8; ++k) hv[k] = p[k];
            } else {
                // block d0 / 128; code j0 + k: low nibble k of the qs bytes from 2 + j0/2, high 2 bits k of the qh
                // bytes from 66 + j0/4 (sj_kvarn.h:1255-1257)
                const uint16_t * b16 = (const uint16_t *) (row + (size_t) (d0 >> 7) * SJKVARN_TQ6_BLOCK_BYTES);
                const int j0 = d0 & 127;
                const uint32_t qs = (uint32_t) b16[1 + j0 / 4] | ((uint32_t) b16[2 + j0 / 4] << 16);
                const uint32_t qh = b16[33 + j0 / 8];
                const float norm = f16_to_f32(b16[0]);
                // a NaN norm gives NaNs of its own sign (the host's product keeps its NaN operand)
                const bool nan_norm = norm != norm;
                const uint16_t nan_h = (uint16_t) ((b16[0] & 0x8000u) | 0x7E00u);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t code = ((qs >> (4 * k)) & 15u) | (((qh >> (2 * k)) & 3u) << 4);
                    hv[k] = nan_norm ? nan_h : f32_to_f16(s.tq6c[code] * norm);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (IS_V) s.M[t * CP + d0 + k] = hv[k];
            else s.M[(d0 + k) * CP + t] = hv[k];
            nf |= (uint32_t) (hv[k] & 0x7FFFu) + 0x400u;
        }
    }
    return nf & 0x8000u;
}

// ------------------------------------------------------------------------------------------------
// balance
// ------------------------------------------------------------------------------------------------

// cur = (M / s_col) / s_row (sj_kvarn.h:980-987). XN: the host's NaN for a NaN input or a NaN scale (the
// dividend's NaN first, then s_col's, then s_row's); the plain form gives the same values and the same NaN-ness.
template <int C, bool XN = false>
SJK_DEV float cur_at(const SealLds & s, int r, int c) {
    const uint16_t h = s.M[r * (C + 2) + c];
    if (XN) {
        const float m = f16_to_f32(h), sc = s.scol[c], sr = s.srow[r];
        if (m != m) return nan_of(m);
        if (sc != sc) return nan_of(sc);
        if (sr != sr) return nan_of(sr);
        return div_by_drecip(div_by_drecip(m, s.ycol[c]), s.yrow[r]);
    }
    const float m = f16_to_f32_fast(h);
    return div_by_drecip(div_by_drecip(m, s.ycol[c]), s.yrow[r]);
}

template <bool XN = false>
SJK_DEV double tree8(const double * p, int stride) {
    if (XN) {
        const double a = xadd(p[0], p[stride]), b = xadd(p[2 * stride], p[3 * stride]);
        const double c = xadd(p[4 * stride], p[5 * stride]), d = xadd(p[6 * stride], p[7 * stride]);
        return xadd(xadd(a, b), xadd(c, d));
    }
    const double a = p[0] + p[stride], b = p[2 * stride] + p[3 * stride];
    const double c = p[4 * stride] + p[5 * stride], d = p[6 * stride] + p[7 * stride];
    return (a + b) + (c + d);
}

// the log-domain scale update of one column (row): clamp the std to [1e-3, 1e3], add its log to the
// accumulator, clamp that to [-0.3, 10], and return the scale (float) exp(acc) (sj_kvarn.h:1000-1002,
// 1006-1008). log and exp are the device's double routines (OCML); sjk_hip_balance_step runs this same
// function on caller arrays so that they can be compared with the host's libm.
// Not inlined: inlined, the compiler hoists the ~30 VGPRs of the double log / exp polynomial constants out of
// the balance loop of the seal, runs out of registers at 1024 threads per workgroup and spills the loop's LDS
// addresses to scratch, reloading them in every pass (232 bytes per lane, ~60 MB of scratch writes per commit).
static __device__ __attribute__((noinline)) float balance_log_step(double & acc, float sd) {
    const float s = tmin(tmax(sd, 1e-3f), 1e3f);
    acc = tmin(tmax(acc + ::log((double) s), -0.3), 10.0);
    return (float) ::exp(acc);
}

__global__ void balance_step_kernel(const float * sd, double * acc, float * scale, int n) {
    const int i = (int) (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    double a = acc[i];
    scale[i] = balance_log_step(a, sd[i]);
    acc[i] = a;
}

// one column pass (COL) or row pass (!COL) of sj_kvarn__balance: sample std of every column (row)
// of cur, then the log-domain update of that column's (row's) scale. XN: the same pass with the host's NaN rule
// (a side holding an infinity or a NaN).
template <int R, int C, bool COL, bool XN>
SJK_DEV void balance_pass(SealLds & s) {
    constexpr int N = COL ? R : C;       // values per reduction
    constexpr int L = N / 8;             // chunk length
    constexpr int NOUT = COL ? C : R;    // reductions in this pass
    constexpr int TPT = 8 * NOUT / SEAL_NT;
    static_assert(TPT >= 1 && TPT * L * SEAL_NT == R * C, "tile/thread mismatch");
    // the thread index is made opaque here so that the pass's LDS addresses are computed in every pass: hoisted
    // over the 2 x iters passes they outnumber the registers left at 1024 threads per workgroup and go to scratch
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    if (XN) {
        // the host's NaN rule; cur is recomputed for the second moment instead of kept in registers (this pass
        // only runs for sides holding an infinity or a NaN)
        for (int tt = 0; tt < TPT; ++tt) {
            const int task = tid + tt * SEAL_NT, o = task % NOUT, k = task / NOUT;
            double acc = 0.0;
#pragma unroll 1
            for (int j = 0; j < L; ++j) {
                const int r = COL ? k * L + j : o, c = COL ? o : k * L + j;
                acc = xadd(acc, f2d_x(cur_at<C, true>(s, r, c)));
            }
            s.u.part.a[k * NOUT + o] = acc;
        }
        __syncthreads();
        for (int tt = 0; tt < TPT; ++tt) {
            const int task = tid + tt * SEAL_NT, o = task % NOUT, k = task / NOUT;
            const double sum = tree8<true>(&s.u.part.a[o], NOUT);
            const double mean = sum != sum ? sum : sum / (double) N;
            double acc = 0.0;
#pragma unroll 1
            for (int j = 0; j < L; ++j) {
                const int r = COL ? k * L + j : o, c = COL ? o : k * L + j;
                const double d = xsub(f2d_x(cur_at<C, true>(s, r, c)), mean);
                acc = d != d ? d : acc != acc ? acc : __builtin_fma(d, d, acc);   // fma(d, d, acc): never invalid
            }
            s.u.part.b[k * NOUT + o] = acc;
        }
        __syncthreads();
    } else {
        float v[TPT][L];
#pragma unroll
        for (int tt = 0; tt < TPT; ++tt) {
            const int task = tid + tt * SEAL_NT, o = task % NOUT, k = task / NOUT;
            double acc = 0.0;
#pragma unroll
            for (int j = 0; j < L; ++j) {
                const int r = COL ? k * L + j : o, c = COL ? o : k * L + j;
                v[tt][j] = cur_at<C>(s, r, c);
                acc = acc + (double) v[tt][j];
            }
            s.u.part.a[k * NOUT + o] = acc;
        }
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TPT; ++tt) {
            const int task = tid + tt * SEAL_NT, o = task % NOUT, k = task / NOUT;
            const double mean = tree8(&s.u.part.a[o], NOUT) / (double) N;
            double acc = 0.0;
#pragma unroll
            for (int j = 0; j < L; ++j) {
                const double d = (double) v[tt][j] - mean;
                acc = __builtin_fma(d, d, acc);
            }
            s.u.part.b[k * NOUT + o] = acc;
        }
        __syncthreads();
    }
    if (tid < NOUT) {
        const double m2 = tree8<XN>(&s.u.part.b[tid], NOUT);
        double * lacc = COL ? s.lcol : s.lrow;
        float sc;
        if (XN && (m2 != m2 || lacc[tid] != lacc[tid])) {
            // a NaN std (or accumulator) passes the clamps and log / exp unchanged: acc + log(s) keeps acc's NaN
            // first, then s's (sj_kvarn.h:1000-1002)
            const double l = lacc[tid] != lacc[tid] ? lacc[tid] : nan_of(m2);
            lacc[tid] = l;
            sc = d2f_x(l);
        } else {
            sc = balance_log_step(lacc[tid], (float) __builtin_sqrt(m2 / (double) (N - 1)));
        }
        (COL ? s.scol : s.srow)[tid] = sc;
        (COL ? s.ycol : s.yrow)[tid] = 1.0 / (double) sc;
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------------------------
// quantize
// ------------------------------------------------------------------------------------------------

SJK_DEV void put_half_g(uint8_t * rec, uint32_t off, float v) {
    *(uint16_t *) (rec + off) = f32_to_f16(v);
}

// per-row lo/hi (sequential-scan semantics of b<a?b:a / a<b?b:a, computed as 8 ordered chunks), the
// step, and the RTN scale/zero halves (sj_kvarn.h:1120-1129)
template <int R, int C, bool IS_V, bool XN>
SJK_DEV void row_affine(const SealArgs & a, SealLds & s, uint8_t * rec) {
    constexpr int L = C / 8, TPT = 8 * R / SEAL_NT;
    const int tid = threadIdx.x;
#pragma unroll
    for (int tt = 0; tt < TPT; ++tt) {
        const int task = tid + tt * SEAL_NT, r = task % R, k = task / R;
        float lo = cur_at<C, XN>(s, r, k * L), hi = lo;
#pragma unroll
        for (int j = 1; j < L; ++j) {
            const float x = cur_at<C, XN>(s, r, k * L + j);
            lo = (lo != lo || x < lo) ? x : lo;   // leftmost minimum of the non-NaN values
            hi = (hi != hi || hi < x) ? x : hi;
        }
        s.u.mm.lo[k * R + r] = lo;
        s.u.mm.hi[k * R + r] = hi;
    }
    __syncthreads();
    if (tid < R) {
        const int r = tid;
        float lo = s.u.mm.lo[r], hi = s.u.mm.hi[r];
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            const float l2 = s.u.mm.lo[k * R + r], h2 = s.u.mm.hi[k * R + r];
            lo = (lo != lo || l2 < lo) ? l2 : lo;
            hi = (hi != hi || hi < h2) ? h2 : hi;
        }
        const float x0 = cur_at<C, XN>(s, r, 0);
        if (x0 != x0) { lo = x0; hi = x0; }   // a NaN first value stays (the reference's scan)
        const int bits = IS_V ? a.lay.bits_v : a.lay.bits_k;
        const float qmax = (float) ((1u << bits) - 1u);
        const float span = XN ? xsub(hi, lo) : hi - lo;            // inf - inf: the host's default NaN
        const float step = tmax(XN && span != span ? span : span / qmax, 1e-10f);
        const uint32_t ri = (uint32_t) (IS_V ? r : k_ch_idx(a.lay, r));
        put_half_g(rec, (IS_V ? a.lay.v_scale : a.lay.k_scale) + 2u * ri, XN ? xmul(s.srow[r], step) : s.srow[r] * step);
        put_half_g(rec, (IS_V ? a.lay.v_zero : a.lay.k_zero) + 2u * ri, XN ? xmul(s.srow[r], lo) : s.srow[r] * lo);
        s.qlo[r] = lo;
        s.qstep[r] = step;
    }
    __syncthreads();
}

// (t, d) of code n (0..7) of payload unit u (8 codes = `bits` bytes at byte u*bits)
template <int D, int G>
SJK_DEV void unit_td(int fmt, bool is_v, int u, int n, int & t, int & d) {
    if (fmt == 0) {            // 4-bit fragment order (sj_kvarn.h:807-833)
        const int tile = u >> 5, wi = u & 31;
        const int tb = tile / (D / 16), db = tile % (D / 16);
        const int aa = (wi >> 2) + 8 * (n & 1);
        const int bb = (n >> 2) + 2 * (wi & 3) + 8 * ((n >> 1) & 1);
        if (!is_v) { t = tb * 16 + aa; d = db * 16 + bb; } else { d = db * 16 + aa; t = tb * 16 + bb; }
    } else if (fmt == 1) {     // token-major
        const int e = u * 8 + n;
        t = e / D; d = e % D;
    } else {                   // channel-major (trellis)
        const int e = u * 8 + n;
        d = e / G; t = e % G;
    }
}

SJK_DEV void store_unit(uint8_t * p, int u, int bits, uint32_t val) {
    if (bits == 4) *(uint32_t *) (p + 4 * u) = val;
    else if (bits == 2) *(uint16_t *) (p + 2 * u) = (uint16_t) val;
    else { p[3 * u] = (uint8_t) val; p[3 * u + 1] = (uint8_t) (val >> 8); p[3 * u + 2] = (uint8_t) (val >> 16); }
}

template <int R, int C, bool IS_V>
SJK_DEV void scalar_codes(const SealArgs & a, SealLds & s, uint8_t * rec) {
    constexpr int D = IS_V ? C : R, G = IS_V ? R : C;
    const int bits = IS_V ? a.lay.bits_v : a.lay.bits_k;
    const int fmt = frag_side(a.lay, bits) ? 0 : 1;
    const float qmax = (float) ((1u << bits) - 1u);
    uint8_t * payload = rec + (IS_V ? a.lay.v_payload : a.lay.k_payload);
    for (int u = threadIdx.x; u < R * C / 8; u += SEAL_NT) {
        uint32_t val = 0;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            int t, d;
            unit_td<D, G>(fmt, IS_V, u, n, t, d);
            const int r = IS_V ? t : d, c = IS_V ? d : t;
            float q = __builtin_rintf((cur_at<C>(s, r, c) - s.qlo[r]) / s.qstep[r]);
            if (q < 0.0f) q = 0.0f;
            if (q > qmax) q = qmax;
            val |= ((uint32_t) q & ((1u << bits) - 1u)) << (n * bits);
        }
        store_unit(payload, u, bits, val);
    }
}

// column scales absorbed into the record: Ktok[t] / Vch[v_ch_idx(d)] (sj_kvarn.h:1141-1146)
template <int R, int C, bool IS_V>
SJK_DEV void col_scales(const SealArgs & a, SealLds & s, uint8_t * rec) {
    const int c = threadIdx.x;
    if (c < C) {
        const uint32_t off = IS_V ? a.lay.v_ch + 2u * (uint32_t) v_ch_idx(a.lay, c) : a.lay.k_tok + 2u * (uint32_t) c;
        put_half_g(rec, off, s.scol[c]);
    }
}

// ------------------------------------------------------------------------------------------------
// trellis
// ------------------------------------------------------------------------------------------------

SJK_DEV float readlane_f(float x, int lane) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane)); }

// 64-state Viterbi of one channel, one state per lane (sj_kvarn.h:1025-1053). y0/y1: target of token
// lane / lane + 64. Returns the codes of tokens lane and lane + 64.
template <int BITS>
SJK_DEV void viterbi_wave(float y0, float y1, const float * cbf, int lane, uint32_t & c0, uint32_t & c1) {
    constexpr int NB = 1 << BITS;
    float cbv[NB];
    int src[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        cbv[j] = cbf[lane + 64 * j];
        src[j] = ((lane + 64 * j) >> BITS) * 4;
    }
    float M = 0.0f;
    uint32_t picks[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) picks[w] = 0;
#pragma unroll
    for (int i = 127; i >= 0; --i) {
        const float yi = readlane_f(i < 64 ? y0 : y1, i & 63);
        float best = __builtin_inff();
        uint32_t pick = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float d = yi - cbv[j];
            const float e = d * d;
            const float mp = __int_as_float(__builtin_amdgcn_ds_bpermute(src[j], __float_as_int(M)));
            const float c = e + mp;
            if (c < best) { best = c; pick = (uint32_t) j; }
        }
        M = best;
        picks[i >> 3] |= pick << (4 * (i & 7));
    }
    int st = 0;
    c0 = 0; c1 = 0;
#pragma unroll
    for (int i = 0; i < 128; ++i) {
        const int pk = (int) ((uint32_t) __builtin_amdgcn_readlane((int) picks[i >> 3], st) >> (4 * (i & 7))) & 15;
        if (i < 64) c0 = lane == i ? (uint32_t) pk : c0;
        else c1 = lane == i - 64 ? (uint32_t) pk : c1;
        st = (st + 64 * pk) >> BITS;
    }
}

template <int R, int C, bool IS_V, int BITS>
SJK_DEV void trellis_side(const SealArgs & a, SealLds & s, uint8_t * rec) {
    constexpr int D = IS_V ? C : R, G = IS_V ? R : C;
    static_assert(G == 128, "trellis sequences are 128 tokens");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Viterbi, one channel per wave at a time
    for (int d = wave; d < D; d += SEAL_NT / 64) {
        float y[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int t = lane + 64 * hh;
            const int r = IS_V ? t : d, c = IS_V ? d : t;
            y[hh] = (cur_at<C>(s, r, c) - s.qlo[r]) / s.qstep[r];
        }
        uint32_t c0, c1;
        viterbi_wave<BITS>(y[0], y[1], s.cbf, lane, c0, c1);
        s.u.codes[d * 128 + lane] = (uint8_t) c0;
        s.u.codes[d * 128 + lane + 64] = (uint8_t) c1;
    }
    __syncthreads();
    // pack channel-major: unit u = 8 tokens of one channel
    uint8_t * payload = rec + (IS_V ? a.lay.v_payload : a.lay.k_payload);
    for (int u = tid; u < D * G / 8; u += SEAL_NT) {
        uint32_t val = 0;
#pragma unroll
        for (int n = 0; n < 8; ++n) val |= (uint32_t) s.u.codes[u * 8 + n] << (n * BITS);
        store_unit(payload, u, BITS, val);
    }
    // moment-matching refit of each row's affine (sj_kvarn.h:1078-1109)
    if (tid < R) {
        const int r = tid;
        double Sx = 0.0, Sy = 0.0, Sxx = 0.0, Syy = 0.0;
        const double n = (double) C;
        for (int c = 0; c < C; ++c) {
            const int ch = IS_V ? c : r, tok = IS_V ? r : c;
            const uint8_t * cd = &s.u.codes[ch * 128];
            uint32_t w = (uint32_t) cd[tok] << 6;
#pragma unroll
            for (int k = 1; k * BITS <= 6; ++k) w |= tok >= k ? (uint32_t) cd[tok - k] << (6 - k * BITS) : 0u;
            const double x = (double) cur_at<C>(s, r, c);
            const double yh = (double) s.cbf[w];
            Sx = Sx + x;
            Sy = Sy + yh;
            Sxx = Sxx + x * x;
            Syy = Syy + yh * yh;
        }
        const double vy = n * Syy - Sy * Sy;
        const double vx = n * Sxx - Sx * Sx;
        if (vy > 0.0 && vx > 0.0) {
            const double ad = __builtin_sqrt(vx / vy);
            const double bd = (Sx - ad * Sy) / n;
            if (ad > 0.0 && bd == bd && !(ad > 1e30) && !(__builtin_fabs(bd) > 1e30)) {
                const uint32_t ri = (uint32_t) (IS_V ? r : k_ch_idx(a.lay, r));
                put_half_g(rec, (IS_V ? a.lay.v_scale : a.lay.k_scale) + 2u * ri, s.srow[r] * (float) ad);
                put_half_g(rec, (IS_V ? a.lay.v_zero : a.lay.k_zero) + 2u * ri, s.srow[r] * (float) bd);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// one side
// ------------------------------------------------------------------------------------------------

template <int R, int C, bool IS_V>
SJK_DEV void seal_side(const SealArgs & a, SealLds & s, int il, int g, int h, uint32_t B_from, uint8_t * rec) {
    const int tid = threadIdx.x;
    if (tid < 64) s.tq6c[tid] = tq6_cent(tid);
    if (a.lay.body == SJKVARN_BODY_TRELLIS) {
        const int bits = IS_V ? a.lay.bits_v : a.lay.bits_k;
        const uint16_t * cb = codebook(bits, IS_V);
        for (int i = tid; i < (1 << (6 + bits)); i += SEAL_NT) s.cbf[i] = f16_to_f32(cb[i]);
    }
    if (tid < C) { s.scol[tid] = 1.0f; s.ycol[tid] = 1.0; s.lcol[tid] = 0.0; }
    if (tid < R) { s.srow[tid] = 1.0f; s.yrow[tid] = 1.0; s.lrow[tid] = 0.0; }
    __syncthreads();
    // a side holding an infinity or a NaN takes the balance and row affine with the host's NaN rule (sjk_dev.h
    // x86_res); finite fp16 inputs make no infinity or NaN anywhere in the seal, so they keep the plain arithmetic
    const int nonfinite = __syncthreads_or((int) load_tile<R, C, IS_V>(a, il, g, h, B_from, s));
    if (nonfinite) {
        for (int it = 0; it < a.iters; ++it) {
            balance_pass<R, C, true, true>(s);
            balance_pass<R, C, false, true>(s);
        }
        row_affine<R, C, IS_V, true>(a, s, rec);
    } else {
        for (int it = 0; it < a.iters; ++it) {
            balance_pass<R, C, true, false>(s);
            balance_pass<R, C, false, false>(s);
        }
        row_affine<R, C, IS_V, false>(a, s, rec);
    }
    if (a.lay.body == SJKVARN_BODY_TRELLIS) {
        const int bits = IS_V ? a.lay.bits_v : a.lay.bits_k;
        if (bits == 3) trellis_side<R, C, IS_V, 3>(a, s, rec);
        else trellis_side<R, C, IS_V, 2>(a, s, rec);
    } else {
        scalar_codes<R, C, IS_V>(a, s, rec);
    }
    col_scales<R, C, IS_V>(a, s, rec);
}

template <int D>
__global__ __launch_bounds__(SEAL_NT) void seal_kernel(SealArgs a) {
    __shared__ SealLds s;
    const int per_layer = a.n_groups * a.H;
    const int il = blockIdx.x / per_layer, rem = blockIdx.x % per_layer;
    const int g = rem / a.H, h = rem % a.H;
    uint8_t * rec;
    uint32_t B_from = a.B_from;
    if (a.desc) {
        // the range of this commit, read at run time; the whole workgroup leaves together (no barrier yet)
        // refused, sealing nothing: negative entries, an empty or misaligned range, and a range of more groups than
        // the launch has (sealing only its first part would leave records that attention reads unsealed)
        const int32_t ib_old = a.desc[SJK_DESC_B_OLD], ib = a.desc[SJK_DESC_B];
        const uint32_t G = (uint32_t) a.lay.G, b_old = (uint32_t) ib_old, b = (uint32_t) ib;
        if (ib_old < 0 || ib < 0 || b <= b_old || b_old < a.S || (b_old - a.S) % G || (b - a.S) % G ||
            (b - b_old) / G > (uint32_t) a.n_groups || (uint32_t) g >= (b - b_old) / G)
            return;
        B_from = b_old;
    }
    if (a.mode == 0) {
        rec = a.body + (size_t) blockIdx.x * a.lay.bytes;
    } else {
        const uint32_t gi = (B_from - a.S) / (uint32_t) a.lay.G + (uint32_t) g;
        const uint32_t blk = a.layers[il].blocks ? a.layers[il].blocks[gi] : gi;
        rec = a.layers[il].body + ((size_t) blk * a.H + h) * a.lay.bytes;
    }
    if (blockIdx.y == 0) seal_side<D, 128, false>(a, s, il, g, h, B_from, rec);
    else seal_side<128, D, true>(a, s, il, g, h, B_from, rec);
}

static int launch_seal(const SealArgs & a, int n_rec, hipStream_t st) {
    if (n_rec <= 0) return 0;
    const dim3 grid((unsigned) n_rec, 2);
    if (a.lay.D == 256) hipLaunchKernelGGL(seal_kernel<256>, grid, dim3(SEAL_NT), 0, st, a);
    else if (a.lay.D == 128) hipLaunchKernelGGL(seal_kernel<128>, grid, dim3(SEAL_NT), 0, st, a);
    else return SJK_ERR_UNSUPPORTED;
    return SJK_CHECK_LAUNCH();
}

}  // namespace sjk

using namespace sjk;

extern "C" int sjk_hip_supported(const sj_kvarn_layout * l) {
    return l && (l->D == 128 || l->D == 256) && l->G == 128 && l->bits_k >= 2 && l->bits_k <= 4 && l->bits_v >= 2 &&
           l->bits_v <= 4 && (l->body == SJKVARN_BODY_SCALAR || l->body == SJKVARN_BODY_TRELLIS);
}

extern "C" int sjk_hip_seal(const sj_kvarn_layout * l, const uint16_t * d_k, const uint16_t * d_v, size_t row_stride,
                            int n_head_kv, int n_groups, int iters, uint8_t * d_body, void * stream) {
    if (!l || !d_k || !d_v || !d_body || n_head_kv <= 0 || n_groups < 0 || iters < 0) return SJKVARN_ERR_ARG;
    if (!sjk_hip_supported(l)) return SJK_ERR_UNSUPPORTED;
    SealArgs a = {};
    a.lay = *l;
    a.iters = iters;
    a.mode = 0;
    a.H = n_head_kv;
    a.n_groups = n_groups;
    a.n_layers = 1;
    a.k = d_k;
    a.v = d_v;
    a.row_stride = row_stride;
    a.body = d_body;
    return launch_seal(a, n_groups * n_head_kv, (hipStream_t) stream);
}

extern "C" int sjk_hip_commit(const sjk_hip_view * views, int n_layers, uint32_t B_from, uint32_t B_to, int iters,
                              void * stream) {
    if (!views || n_layers <= 0 || iters < 0) return SJKVARN_ERR_ARG;
    if (n_layers > SEAL_MAX_LAYERS) return SJK_ERR_UNSUPPORTED;
    const sjk_hip_view & v0 = views[0];
    const uint32_t G = (uint32_t) v0.lay.G;
    if (B_to <= B_from) return 0;
    if (B_from < v0.S || (B_from - v0.S) % G || (B_to - v0.S) % G) return SJKVARN_ERR_ARG;
    if (!sjk_hip_supported(&v0.lay)) return SJK_ERR_UNSUPPORTED;
    SealArgs a = {};
    a.lay = v0.lay;
    a.iters = iters;
    a.mode = 1;
    a.H = v0.n_head_kv;
    a.n_groups = (int) ((B_to - B_from) / G);
    a.n_layers = n_layers;
    a.staging = v0.staging;
    a.S = v0.S;
    a.cap = v0.cap;
    a.B_from = B_from;
    a.stage_bytes = v0.stage_bytes;
    for (int i = 0; i < n_layers; ++i) {
        const sjk_hip_view & v = views[i];
        if (v.lay.bytes != v0.lay.bytes || v.lay.body != v0.lay.body || v.n_head_kv != v0.n_head_kv || v.S != v0.S ||
            v.cap != v0.cap || v.staging != v0.staging || !v.ring || !v.body)
            return SJKVARN_ERR_ARG;
        a.layers[i].ring = v.ring;
        a.layers[i].body = v.body;
        a.layers[i].blocks = v.blocks;
    }
    return launch_seal(a, n_layers * a.n_groups * a.H, (hipStream_t) stream);
}

// sjk_hip_commit with the range read on the device (the fixed-size launch of the reference's seal_dyn)
extern "C" int sjk_hip_commit_dyn(const sjk_hip_view * views, int n_layers, const int32_t * d_desc, int n_groups_max,
                                  int iters, void * stream) {
    if (!views || !d_desc || n_layers <= 0 || n_groups_max < 0 || iters < 0) return SJKVARN_ERR_ARG;
    if (n_layers > SEAL_MAX_LAYERS) return SJK_ERR_UNSUPPORTED;
    const sjk_hip_view & v0 = views[0];
    if (!sjk_hip_supported(&v0.lay)) return SJK_ERR_UNSUPPORTED;
    if (v0.cap == 0) return SJKVARN_ERR_ARG;
    SealArgs a = {};
    a.lay = v0.lay;
    a.iters = iters;
    a.mode = 1;
    a.H = v0.n_head_kv;
    a.n_groups = n_groups_max;                   // launch size; groups past the descriptor's range leave at once
    a.n_layers = n_layers;
    a.staging = v0.staging;
    a.S = v0.S;
    a.cap = v0.cap;
    a.stage_bytes = v0.stage_bytes;
    a.desc = d_desc;
    for (int i = 0; i < n_layers; ++i) {
        const sjk_hip_view & v = views[i];
        if (v.lay.bytes != v0.lay.bytes || v.lay.body != v0.lay.body || v.n_head_kv != v0.n_head_kv || v.S != v0.S ||
            v.cap != v0.cap || v.staging != v0.staging || !v.ring || !v.body)
            return SJKVARN_ERR_ARG;
        a.layers[i].ring = v.ring;
        a.layers[i].body = v.body;
        a.layers[i].blocks = v.blocks;
    }
    return launch_seal(a, n_layers * n_groups_max * a.H, (hipStream_t) stream);
}

extern "C" int sjk_hip_balance_step(const float * d_sd, double * d_acc, float * d_scale, int n, void * stream) {
    if (!d_sd || !d_acc || !d_scale || n < 0) return SJKVARN_ERR_ARG;
    if (!n) return 0;
    hipLaunchKernelGGL(sjk::balance_step_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, (hipStream_t) stream,
                       d_sd, d_acc, d_scale, n);
    return SJK_CHECK_LAUNCH();
}
