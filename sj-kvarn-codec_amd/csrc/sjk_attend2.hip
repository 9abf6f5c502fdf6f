// sjk_attend2.hip - streaming decode attention on the matrix cores (4-bit scalar body, D = 256).
//
// The context of each KV head is cut into 128-position chunks: fp16 sink chunks, one chunk per sealed
// record, and staging-tail chunks (tq6_0 or fp16 rows of the ring). A workgroup (4 wavefronts) walks a
// contiguous run of chunks of ONE kind for all query rows of its KV head (decode width x GQA group
// <= 16): "record" workgroups stream sealed records, "row" workgroups take the sink and the tail. The
// two kinds are separate kernels so that each gets its own register allocation.
// Per chunk every wavefront owns 32 positions and keeps its own online softmax (m, l) and O[16][256]
// in registers; the four are merged once at the end into one partial (m, l, O) per workgroup, and
// attend_combine2 merges the partials with the log-sum-exp rule.
//
// Sealed records go through v_mfma_f32_16x16x32_f16 without dequantizing the payload:
//   K[t,d] = (c*Kscale[d] + Kzero[d]) * Ktok[t]  ->  S[q,t] = Ktok[t] * (sum_d Q'[q,d]*c[t,d] + sum_d Q[q,d]*Kzero[d]),
//   with Q' = Q * Kscale (per record), and
//   V[t,d] = (c*Vscale[t] + Vzero[t]) * Vch[d]   ->  O[q,d] += Vch[d] * (sum_t P'[q,t]*c[t,d] + sum_t P[q,t]*Vzero[t]),
//   with P' = P * Vscale. The codes c (0..15) enter the MFMA as exact fp16 values 16 + c, built from the
//   record's 16x16-tile fragment words with one rotate and one and-or per two codes; the +16 is
//   removed through the same correction terms. Q' and P' are split into fp16 hi + lo parts (two
//   MFMAs), which keeps ~22 significant bits, so the products stay within fp32-accumulation error of
//   the reference's fp32 dot products (sj_kvarn.h:1288-1311; bar: 1e-3 abs / rel on the output).
// The k-order of each MFMA is a permutation chosen so that (a) one 8-byte LDS read per lane yields a
// full operand and (b) the QK accumulator (rows = tokens 4g+i of two 16-token tiles, column = query)
// is already the A operand of the PV product: no transpose, no LDS round trip for P.
// Sink and tail rows use exact values instead (fp16, or tq6_0 centroid * block norm as the reference
// dequantizes them, sj_kvarn.h:1249-1260), split hi + lo, with three MFMAs per product.
#include "sjk_dev.h"

namespace sjk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int A2_NT = 256;      // 4 wavefronts
constexpr int A2_Q = 16;        // query rows per KV head
constexpr int A2_D = 256;

// record layout of the 4/4 scalar body at D = 256, G = 128 (sj_kvarn.h:771-790), as constants so every
// LDS address below is a base register plus an immediate offset
constexpr int R_VPAY = 16384, R_KSC = 32768, R_KZE = 33280, R_KTOK = 33792, R_VCH = 34048, R_VSC = 34560,
              R_VZE = 34816, R_BYTES = 35072;
// channel index of the per-channel K / V scales (fragment order, sj_kvarn.h:835-849) at D = 256
SJK_DEV constexpr int a2_kci(int d) { return ((d >> 1) & 3) * 64 + (d >> 4) * 4 + ((d >> 3) & 1) * 2 + (d & 1); }
SJK_DEV constexpr int a2_vci(int d) { return (d & 7) * 32 + (d >> 4) * 2 + ((d >> 3) & 1); }

struct Att2Args {
    sjk_hip_view v;
    uint32_t B, N, qpos0;
    int n_q, n_head, gq, n_rows;
    float scale;
    const float * q;
    float * out;
    float * part;                 // [H][n_wg][A2_Q][A2_D + 2]
    uint32_t sink_end, body_end, pend;
    int sink_chunks, body_chunks, tail_chunks;
    int row_per_wg, rec_per_wg;   // chunks per workgroup
    int n_row_wg, n_rec_wg, n_wg; // workgroups per KV head: row kind first, then record kind
};

struct Att2Lds {
    alignas(16) uint8_t rec[R_BYTES];          // one record (record chunks) / row staging / O merge buffer
    alignas(16) uint16_t qb[2][8][4][A2_Q][8];  // Q' (records) or Q (rows), hi / lo, B-operand order
    float corr[A2_Q];                          // records: 16*sum Q' - sum Q*Kzero per query
    float wm[4][A2_Q], wl[4][A2_Q];            // per-wave softmax state at the merge
};

// hi / lo fp16 split of x: hi = RN16(x), lo = RN16(x - hi) (x - hi is exact in fp32)
SJK_DEV void split_hl(float x, uint32_t & hi, uint32_t & lo) {
    const _Float16 h = (_Float16) x;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16) (x - (float) h));
}

SJK_DEV uint32_t pack2(uint32_t a, uint32_t b) { return a | (b << 16); }

// two codes (nibbles b and b+4 of w) as the fp16 pair (16 + c_b, 16 + c_{b+4})
SJK_DEV uint32_t code_pair(uint32_t w, uint32_t rot) {
    return (__builtin_amdgcn_alignbit(w, w, rot) & 0x03C003C0u) | 0x4C004C00u;
}

SJK_DEV f4 mfma(const u4 & a, const u4 & b, const f4 & c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

// B-operand position of channel d: (k-step s, group g, slot i), the inverse of slot_chan
SJK_DEV void chan_slot(int d, int & s, int & g, int & i) {
    const int db = d >> 4, dd = d & 15;
    s = db >> 1;
    g = 2 * (db & 1) + ((dd & 7) >> 2);
    i = 4 * ((dd >> 1) & 1) + 2 * (dd >> 3) + (dd & 1);
}

SJK_DEV int slot_chan(int s, int g, int i) {
    return 16 * (2 * s + (g >> 1)) + 4 * (g & 1) + 2 * (i >> 2) + (i & 1) + 8 * ((i >> 1) & 1);
}

SJK_DEV float half_at(const uint8_t * p) { return f16_to_f32_fast(*(const uint16_t *) p); }

// LDS writes of this wavefront visible to its other lanes
SJK_DEV void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// K (side 0) or V (side 1) row of position p, KV head h: the sink (p < S) or the staging ring
SJK_DEV const uint8_t * value_row(const sjk_hip_view & V, uint32_t p, int h, int side) {
    const int H = V.n_head_kv;
    if (p < V.S && V.sink_type == SJKVARN_SINK_F16) return V.sink + ((size_t) p * H + h) * 4 * A2_D + side * 2 * A2_D;
    const uint8_t * e = p < V.S ? V.sink + ((size_t) p * H + h) * 2 * V.stage_bytes
                                : V.ring + ((size_t) ((p - V.S) % V.cap) * H + h) * 2 * V.stage_bytes;
    return e + side * V.stage_bytes;
}

SJK_DEV bool value_f16(const sjk_hip_view & V, bool sink) {
    return (sink && V.sink_type == SJKVARN_SINK_F16) || V.staging == SJKVARN_STAGING_F16;
}

// values of channels d, d+1 (d even) of a row: fp16, or tq6_0 centroid * block norm
SJK_DEV void value_pair(const uint8_t * row, bool f16row, int d, float norm, float & x0, float & x1) {
    if (f16row) {
        const uint32_t v = *(const uint32_t *) (row + 2 * d);
        x0 = f16_to_f32_fast((uint16_t) v);
        x1 = f16_to_f32_fast((uint16_t) (v >> 16));
        return;
    }
    const uint8_t * blk = row + (d >> 7) * SJKVARN_TQ6_BLOCK_BYTES;
    const int j = d & 127;
    const uint32_t qs = blk[2 + (j >> 1)], qh = blk[66 + (j >> 2)] >> (2 * (j & 3));
    x0 = tq6_cent((int) ((qs & 15u) | ((qh & 3u) << 4))) * norm;
    x1 = tq6_cent((int) ((qs >> 4) | (((qh >> 2) & 3u) << 4))) * norm;
}

// query rows of this KV head: thread (cq = tid/16, cb = tid%16) holds Q[cq][16cb .. 16cb+15]
SJK_DEV void load_q(const Att2Args & a, int h, float * qv) {
    const int tid = threadIdx.x, cq = tid >> 4, cb = tid & 15;
    const bool live = cq < a.n_rows;
    const int iq = live ? cq / a.gq : 0, hq = h * a.gq + (live ? cq % a.gq : 0);
    const float * src = a.q + ((size_t) iq * a.n_head + hq) * A2_D + 16 * cb;
#pragma unroll
    for (int k = 0; k < 16; ++k) qv[k] = live ? src[k] : 0.0f;
}

// online-softmax update of this wave for its 8 scores; returns alpha (rescale of the old state)
SJK_DEV float softmax_step(float * sc, float & m_run, float & l_run) {
    float mloc = sc[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) mloc = fmaxf(mloc, sc[k]);
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const bool any = m_new != -__builtin_inff();
    const float alpha = any ? __expf(m_run - m_new) : 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        sc[k] = any ? __expf(sc[k] - m_new) : 0.0f;
        psum += sc[k];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    m_run = m_new;
    l_run = l_run * alpha + psum;
    return alpha;
}

// merge the four wavefronts' (m, l, O) and write the workgroup partial
SJK_DEV void write_partial(const Att2Args & a, Att2Lds & s, int h, int wgi, const f4 * O, float m_run, float l_run) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    __syncthreads();
    if (g == 0) { s.wm[w][n] = m_run; s.wl[w][n] = l_run; }
    __syncthreads();
    float fac[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * g + i;
        const float M = fmaxf(fmaxf(s.wm[0][q], s.wm[1][q]), fmaxf(s.wm[2][q], s.wm[3][q]));
        fac[i] = M == -__builtin_inff() ? 0.0f : __expf(s.wm[w][q] - M);
    }
    float * ob = (float *) s.rec;     // [16][256]
    for (int k = 0; k < 4; ++k) {
        if (w == k) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float & dst = ob[(4 * g + i) * A2_D + 16 * j + n];
                    dst = (k == 0 ? 0.0f : dst) + O[j][i] * fac[i];
                }
        }
        __syncthreads();
    }
    float * part = a.part + ((size_t) h * a.n_wg + wgi) * A2_Q * (A2_D + 2);
    for (int e = tid; e < A2_Q * A2_D; e += A2_NT) part[(e / A2_D) * (A2_D + 2) + 2 + (e % A2_D)] = ob[e];
    if (tid < A2_Q) {
        const float M = fmaxf(fmaxf(s.wm[0][tid], s.wm[1][tid]), fmaxf(s.wm[2][tid], s.wm[3][tid]));
        float Ls = 0.0f;
        if (M != -__builtin_inff())
            for (int k = 0; k < 4; ++k) Ls += s.wl[k][tid] * __expf(s.wm[k][tid] - M);
        part[tid * (A2_D + 2)] = M;
        part[tid * (A2_D + 2) + 1] = Ls;
    }
}

// ------------------------------------------------------------------------------------------------
// record workgroups
// ------------------------------------------------------------------------------------------------

__device__ __attribute__((always_inline)) inline void a2_records(const Att2Args & a, Att2Lds & s, int h, int r0, int r1, int wgi) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    const sjk_hip_view & V = a.v;
    const int H = V.n_head_kv;
    const int cq = tid >> 4, cb = tid & 15;
    float qv[16];
    load_q(a, h, qv);
    const uint32_t qpos = a.qpos0 + (uint32_t) (n < a.n_rows ? n / a.gq : 0);
    const uint32_t qend = n < a.n_rows ? (qpos + 1 < a.N ? qpos + 1 : a.N) : 0u;
    float m_run = -__builtin_inff(), l_run = 0.0f;
    f4 O[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // per-lane operand addresses inside a staged record
    const uint32_t kword = (uint32_t) (4 * (n & 7) + 2 * (g & 1)) * 4u;
    const uint32_t kb = (uint32_t) (n >> 3), vb = (uint32_t) ((n >> 3) + 2 * (g >> 1));
    const uint32_t rk0 = (4u * kb - 6u) & 31u, rk1 = (4u * kb + 2u) & 31u, rv = (4u * vb - 6u) & 31u;

    // the next record's bytes are loaded into registers while the current one is computed:
    // thread tid holds 16-byte vectors tid + 256 k of the record (2192 vectors)
    constexpr int NV = R_BYTES / 16, PF = (NV + A2_NT - 1) / A2_NT;
    u4 pf[PF];
    auto fetch = [&](int c) {
        const uint32_t gi = (a.sink_end + (uint32_t) c * 128u - V.S) / 128u;
        const uint32_t blk = V.blocks ? V.blocks[gi] : gi;
        const u4 * src = (const u4 *) (V.body + ((size_t) blk * H + h) * R_BYTES);
#pragma unroll
        for (int k = 0; k < PF; ++k)
            if (tid + A2_NT * k < NV) pf[k] = src[tid + A2_NT * k];
    };
    if (r0 < r1) fetch(r0);

    for (int c = r0; c < r1; ++c) {
        const uint32_t p0 = a.sink_end + (uint32_t) c * 128u;
        __syncthreads();     // the previous record's readers are done
        {
            u4 * dst = (u4 *) s.rec;
#pragma unroll
            for (int k = 0; k < PF; ++k)
                if (tid + A2_NT * k < NV) dst[tid + A2_NT * k] = pf[k];
        }
        if (c + 1 < r1) fetch(c + 1);
        __builtin_amdgcn_sched_barrier(0);   // all prefetch loads issue here, before the compute
        __syncthreads();
        // Q' = Q * Kscale (hi / lo, B-operand order) and the per-query correction
        {
            float corr = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int d = 16 * cb + k;
                const int ci = a2_kci(d);
                const float ks = half_at(s.rec + R_KSC + 2 * ci), kz = half_at(s.rec + R_KZE + 2 * ci);
                const float qq = qv[k] * ks;
                uint32_t hi, lo;
                split_hl(qq, hi, lo);
                int ss, gg, ii;
                chan_slot(d, ss, gg, ii);
                s.qb[0][ss][gg][cq][ii] = (uint16_t) hi;
                s.qb[1][ss][gg][cq][ii] = (uint16_t) lo;
                corr = corr + (16.0f * qq - qv[k] * kz);
            }
            corr += __shfl_xor(corr, 1, 64);
            corr += __shfl_xor(corr, 2, 64);
            corr += __shfl_xor(corr, 4, 64);
            corr += __shfl_xor(corr, 8, 64);
            if (cb == 0) s.corr[cq] = corr;
        }
        __syncthreads();
        // scores of this wave's 32 tokens (two 16-token tiles)
        f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
#pragma unroll 2
        for (int ks = 0; ks < 8; ++ks) {
            const u4 Bh = *(const u4 *) &s.qb[0][ks][g][n][0];
            const u4 Bl = *(const u4 *) &s.qb[1][ks][g][n][0];
            const int db = 2 * ks + (g >> 1);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const uint2 wd = *(const uint2 *) (s.rec + ((2 * w + tt) * 16 + db) * 128 + kword);
                const u4 A = u4{code_pair(wd.x, rk0), code_pair(wd.x, rk1), code_pair(wd.y, rk0), code_pair(wd.y, rk1)};
                acc[tt] = mfma(A, Bh, acc[tt]);
                acc[tt] = mfma(A, Bl, acc[tt]);
            }
        }
        float sc[8];
        const float cq_corr = s.corr[n];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = 32 * w + 16 * tt + 4 * g + i;
                const float raw = half_at(s.rec + R_KTOK + 2 * tok) * (acc[tt][i] - cq_corr);
                sc[4 * tt + i] = p0 + (uint32_t) tok < qend ? raw * a.scale : -__builtin_inff();
            }
        const float alpha = softmax_step(sc, m_run, l_run);
        float arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * g + i, 64);
        // P' = P * Vscale (hi / lo), corrV = sum P*Vzero - 16 sum P'
        u4 Ah, Al;
        float cv = 0.0f;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            uint32_t hh[2], ll[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int k = 2 * pr + e;
                const int tok = 32 * w + 16 * (k >> 2) + 4 * g + (k & 3);
                const float pp = sc[k] * half_at(s.rec + R_VSC + 2 * tok);
                split_hl(pp, hh[e], ll[e]);
                cv = cv + (sc[k] * half_at(s.rec + R_VZE + 2 * tok) - 16.0f * pp);
            }
            Ah[pr] = pack2(hh[0], hh[1]);
            Al[pr] = pack2(ll[0], ll[1]);
        }
        cv += __shfl_xor(cv, 16, 64);
        cv += __shfl_xor(cv, 32, 64);
        // the correction enters as the accumulator input: t = sum P'(16 + c) + corrV
        f4 crow;
#pragma unroll
        for (int i = 0; i < 4; ++i) crow[i] = __shfl(cv, 4 * g + i, 64);
        // rows whose running maximum did not move keep alpha == 1: skip the rescale (wave-uniform test)
        const bool rescale = __any(arow[0] != 1.0f || arow[1] != 1.0f || arow[2] != 1.0f || arow[3] != 1.0f);
        if (rescale) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) O[j][i] = O[j][i] * arow[i];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint2 w0 = *(const uint2 *) (s.rec + R_VPAY + ((2 * w) * 16 + j) * 128 + kword);
            const uint2 w1 = *(const uint2 *) (s.rec + R_VPAY + ((2 * w + 1) * 16 + j) * 128 + kword);
            const u4 Bv = u4{code_pair(w0.x, rv), code_pair(w0.y, rv), code_pair(w1.x, rv), code_pair(w1.y, rv)};
            f4 t = mfma(Ah, Bv, crow);
            t = mfma(Al, Bv, t);
            const float vch = half_at(s.rec + R_VCH + 2 * a2_vci(16 * j + n));
#pragma unroll
            for (int i = 0; i < 4; ++i) O[j][i] = __builtin_fmaf(vch, t[i], O[j][i]);
            __builtin_amdgcn_sched_barrier(0);   // one tile's operands live at a time
        }
    }
    write_partial(a, s, h, wgi, O, m_run, l_run);
}

// ------------------------------------------------------------------------------------------------
// row workgroups: sink and staging tail. One wavefront per 32 positions; the chunk's raw K|V rows are
// staged in LDS with 8-byte loads (all in flight together), values are decoded from LDS as exact
// fp16 hi + lo parts (fp16 rows: the value; tq6_0 rows: the centroid, with the block norm applied to
// the accumulator for K and folded into P for V), three MFMAs per product.
// The k-slot order of this path is contiguous: slot i of group g at k-step ks is channel 32 ks + 8 g + i.
// ------------------------------------------------------------------------------------------------

constexpr int RW_POS = 32;      // positions staged at a time
constexpr int RW_SPAN = 128;    // positions per row wavefront

struct RowLds {
    alignas(16) uint8_t rows[RW_POS * 1024];   // staged K|V rows (stride 2*stage_bytes, or 1 KB for fp16 sinks)
    alignas(16) uint16_t stg[2][4][16][8];     // V operand transpose [hl][g][channel][slot]
    uint32_t cent_hl[64];                      // tq6_0 centroid as fp16 hi | lo << 16
};

// channels c..c+7 (c % 8 == 0) of a staged row as fp16 hi / lo operand quads
SJK_DEV void row8(const uint8_t * row, bool f16row, int c, const uint32_t * cent_hl, u4 & hi, u4 & lo) {
    if (f16row) {
        hi = *(const u4 *) (row + 2 * c);
        lo = u4{0, 0, 0, 0};
        return;
    }
    const uint8_t * blk = row + (c >> 7) * SJKVARN_TQ6_BLOCK_BYTES;
    const int j = c & 127;
    const uint32_t qs = (uint32_t) *(const uint16_t *) (blk + 2 + j / 2) | ((uint32_t) *(const uint16_t *) (blk + 4 + j / 2) << 16);
    const uint32_t qh = *(const uint16_t *) (blk + 66 + j / 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t c0 = ((qs >> (8 * e)) & 15u) | (((qh >> (4 * e)) & 3u) << 4);
        const uint32_t c1 = ((qs >> (8 * e + 4)) & 15u) | (((qh >> (4 * e + 2)) & 3u) << 4);
        const uint32_t t0 = cent_hl[c0], t1 = cent_hl[c1];
        hi[e] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
        lo[e] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
    }
}

__global__ __launch_bounds__(64) void attend2_rows_kernel(Att2Args a) {
    __shared__ RowLds s;
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const int h = blockIdx.y, c = blockIdx.x;
    const sjk_hip_view & V = a.v;
    // this wavefront's run of positions: up to RW_SPAN positions of the sink or of the tail
    const int sinkn = (int) ((a.sink_end + RW_SPAN - 1) / RW_SPAN);
    const bool sink = c < sinkn;
    uint32_t p0, p1;
    if (sink) { p0 = (uint32_t) c * RW_SPAN; p1 = p0 + RW_SPAN < a.sink_end ? p0 + RW_SPAN : a.sink_end; }
    else { p0 = a.body_end + (uint32_t) (c - sinkn) * RW_SPAN; p1 = p0 + RW_SPAN < a.pend ? p0 + RW_SPAN : a.pend; }
    const bool f16row = value_f16(V, sink);
    const bool sinkf16 = sink && V.sink_type == SJKVARN_SINK_F16;
    const int RS = sinkf16 ? 4 * A2_D : (int) (2 * V.stage_bytes);       // staged row stride: K | V
    const int VOFF = sinkf16 ? 2 * A2_D : (int) V.stage_bytes;           // V part inside a staged row
    {
        uint32_t hi, lo;
        split_hl(tq6_cent(lane), hi, lo);
        s.cent_hl[lane] = hi | (lo << 16);
    }
    // Q of query row n, channels of this lane's k-slots, split hi / lo (B operands of the 8 k-steps)
    u4 Bh[8], Bl[8];
    {
        const bool live = n < a.n_rows;
        const int iq = live ? n / a.gq : 0, hq = h * a.gq + (live ? n % a.gq : 0);
        const float * qr = a.q + ((size_t) iq * a.n_head + hq) * A2_D;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const float4 x0 = *(const float4 *) (qr + 32 * ks + 8 * g), x1 = *(const float4 *) (qr + 32 * ks + 8 * g + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t h0, l0, h1, l1;
                split_hl(live ? xv[2 * e] : 0.0f, h0, l0);
                split_hl(live ? xv[2 * e + 1] : 0.0f, h1, l1);
                Bh[ks][e] = pack2(h0, h1);
                Bl[ks][e] = pack2(l0, l1);
            }
        }
    }
    const uint32_t qpos = a.qpos0 + (uint32_t) (n < a.n_rows ? n / a.gq : 0);
    const uint32_t qend = n < a.n_rows ? (qpos + 1 < a.N ? qpos + 1 : a.N) : 0u;
    const int tk = lane >> 1, ch8 = 8 * (lane & 1);                     // transpose writer role
    const int wgr = (tk & 15) >> 2, wsl = 4 * (tk >> 4) + (tk & 3);
    float m_run = -__builtin_inff(), l_run = 0.0f;
    f4 O[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t q0 = p0; q0 < p1; q0 += RW_POS) {
        const uint32_t q1 = q0 + RW_POS < p1 ? q0 + RW_POS : p1;
        __syncthreads();     // the previous sub-chunk's readers are done
        // stage the rows (positions past q1 repeat row q0: finite values, masked below), eight 8-byte
        // loads in flight per lane before their LDS writes
        {
            const int words = RS / 8, total = RW_POS * words;
            for (int e0 = lane; e0 < total; e0 += 64 * 8) {
                uint2 v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int e = e0 + 64 * k;
                    if (e < total) {
                        const int r = e / words, wd = e % words;
                        const uint32_t p = q0 + (uint32_t) r < q1 ? q0 + (uint32_t) r : q0;
                        v[k] = *(const uint2 *) (value_row(V, p, h, 0) + 8 * wd);
                    }
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int e = e0 + 64 * k;
                    if (e < total) *(uint2 *) (s.rows + (e / words) * RS + 8 * (e % words)) = v[k];
                }
            }
        }
        __syncthreads();
        // scores: A = K values of token n of each 16-token tile; tq6 blocks accumulate separately
        f4 acc[2][2] = {{f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}, {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                u4 Ah, Al;
                row8(s.rows + (16 * tt + n) * RS, f16row, 32 * ks + 8 * g, s.cent_hl, Ah, Al);
                f4 & dst = acc[tt][ks >> 2];
                dst = mfma(Ah, Bh[ks], dst);
                dst = mfma(Ah, Bl[ks], dst);
                if (!f16row) dst = mfma(Al, Bh[ks], dst);
            }
        }
        float sc[8];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * tt + 4 * g + i;
                const uint8_t * row = s.rows + r * RS;
                const float raw = f16row ? acc[tt][0][i] + acc[tt][1][i]
                                         : half_at(row) * acc[tt][0][i] + half_at(row + SJKVARN_TQ6_BLOCK_BYTES) * acc[tt][1][i];
                const uint32_t p = q0 + (uint32_t) r;
                sc[4 * tt + i] = (p < q1 && p < qend) ? raw * a.scale : -__builtin_inff();
            }
        const float alpha = softmax_step(sc, m_run, l_run);
        float arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) O[j][i] = O[j][i] * arow[i];
        // A operands of the PV products: P (fp16 rows) or P * block norm (tq6_0 rows, per 128-channel block)
        u4 Ah[2], Al[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                uint32_t hh[2], ll[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int k = 2 * pr + e;
                    const int r = 16 * (k >> 2) + 4 * g + (k & 3);
                    const float nrm = f16row ? 1.0f : half_at(s.rows + r * RS + VOFF + b * SJKVARN_TQ6_BLOCK_BYTES);
                    split_hl(sc[k] * nrm, hh[e], ll[e]);
                }
                Ah[b][pr] = pack2(hh[0], hh[1]);
                Al[b][pr] = pack2(ll[0], ll[1]);
            }
        // V through the LDS transpose: writer lane = (token tk, channels ch8..ch8+7 of the tile),
        // reader lane = (channel n, token slots of g)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            u4 vh, vl;
            row8(s.rows + tk * RS + VOFF, f16row, 16 * j + ch8, s.cent_hl, vh, vl);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s.stg[0][wgr][ch8 + 2 * e][wsl] = (uint16_t) vh[e];
                s.stg[0][wgr][ch8 + 2 * e + 1][wsl] = (uint16_t) (vh[e] >> 16);
                s.stg[1][wgr][ch8 + 2 * e][wsl] = (uint16_t) vl[e];
                s.stg[1][wgr][ch8 + 2 * e + 1][wsl] = (uint16_t) (vl[e] >> 16);
            }
            wave_sync();
            const u4 Vh = *(const u4 *) &s.stg[0][g][n][0];
            const u4 Vl = *(const u4 *) &s.stg[1][g][n][0];
            wave_sync();
            const int b = j >> 3;
            O[j] = mfma(Ah[b], Vh, O[j]);
            O[j] = mfma(Al[b], Vh, O[j]);
            if (!f16row) O[j] = mfma(Ah[b], Vl, O[j]);
        }
    }
    float * part = a.part + ((size_t) h * a.n_wg + c) * A2_Q * (A2_D + 2);
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[(4 * g + i) * (A2_D + 2) + 2 + 16 * j + n] = O[j][i];
    if (g == 0) { part[n * (A2_D + 2)] = m_run; part[n * (A2_D + 2) + 1] = l_run; }
}

// record workgroups: partial slots [n_row_wg, n_wg)
__global__ __launch_bounds__(A2_NT) __attribute__((amdgpu_waves_per_eu(2))) void attend2_records_kernel(Att2Args a) {
    __shared__ Att2Lds s;
    const int h = blockIdx.y, wg = blockIdx.x;
    const int r0 = wg * a.rec_per_wg;
    a2_records(a, s, h, r0, r0 + a.rec_per_wg < a.body_chunks ? r0 + a.rec_per_wg : a.body_chunks, a.n_row_wg + wg);
}

// log-sum-exp merge of the workgroup partials: one wavefront per (query row, KV head, 64 channels)
constexpr int A2_CMB_MAX = 4096;   // partials per KV head the combine holds in LDS

__global__ __launch_bounds__(64) void attend_combine2(Att2Args a) {
    __shared__ float s_w[A2_CMB_MAX];
    const int qi = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, d = blockIdx.z * 64 + lane;
    if (qi >= a.n_rows) return;
    const size_t stride = (size_t) A2_Q * (A2_D + 2);
    const float * base = a.part + (size_t) h * a.n_wg * stride + qi * (A2_D + 2);
    float M = -__builtin_inff();
    for (int c = lane; c < a.n_wg; c += 64) M = fmaxf(M, base[c * stride]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    float Ls = 0.0f;
    for (int c = lane; c < a.n_wg; c += 64) {
        const float m = base[c * stride];
        const float f = (M == -__builtin_inff() || m == -__builtin_inff()) ? 0.0f : __expf(m - M);
        s_w[c] = f;
        Ls += f * base[c * stride + 1];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) Ls += __shfl_xor(Ls, o, 64);
    __syncthreads();
    float o8[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int c = 0;
    for (; c + 8 <= a.n_wg; c += 8) {
        float x[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = base[(size_t) (c + k) * stride + 2 + d];
#pragma unroll
        for (int k = 0; k < 8; ++k) o8[k] += s_w[c + k] * x[k];
    }
    for (; c < a.n_wg; ++c) o8[0] += s_w[c] * base[(size_t) c * stride + 2 + d];
    const float Os = ((o8[0] + o8[1]) + (o8[2] + o8[3])) + ((o8[4] + o8[5]) + (o8[6] + o8[7]));
    const int iq = qi / a.gq, hq = h * a.gq + qi % a.gq;
    a.out[((size_t) iq * a.n_head + hq) * A2_D + d] = Ls == 0.0f ? 0.0f : Os / Ls;
}

}  // namespace sjk

using namespace sjk;

static float * g_part2 = nullptr;
static size_t g_part2_bytes = 0;

// 1 when the streaming kernel handles this view (else the generic kernel in sjk_attend.hip runs)
extern "C" int sjk_attend2_supported(const sjk_hip_view * v, int n_rows) {
    const sj_kvarn_layout & l = v->lay;
    return l.D == 256 && l.G == 128 && l.body == SJKVARN_BODY_SCALAR && l.bits_k == 4 && l.bits_v == 4 &&
           l.bytes == (uint32_t) R_BYTES && l.v_payload == (uint32_t) R_VPAY && l.v_ch == (uint32_t) R_VCH &&
           v->S % 64 == 0 && n_rows <= A2_Q;
}

extern "C" int sjk_attend2(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                           const float * d_q, float scale, float * d_out, void * stream) {
    Att2Args a = {};
    a.v = *v;
    a.B = B; a.N = N; a.qpos0 = qpos0; a.n_q = n_q; a.n_head = n_head;
    a.gq = n_head / v->n_head_kv;
    a.n_rows = n_q * a.gq;
    a.scale = scale; a.q = d_q; a.out = d_out;
    const uint32_t last = qpos0 + (uint32_t) n_q;
    a.pend = N < last ? N : last;
    const uint32_t S = v->S;
    a.sink_end = a.pend < S ? a.pend : S;
    // sealed groups up to the one holding the last visible position (later groups are not read; the
    // positions of that group past it are masked)
    uint32_t Bb = B < S ? S : B;
    const uint32_t pend_g = a.pend <= S ? S : S + (a.pend - S + 127u) / 128u * 128u;
    if (Bb > pend_g) Bb = pend_g;
    a.body_end = Bb;
    a.sink_chunks = (int) ((a.sink_end + 127) / 128);
    a.body_chunks = (int) ((a.body_end - S) / 128);
    a.tail_chunks = (int) ((a.pend > a.body_end ? a.pend - a.body_end + 127 : 0) / 128);
    const int H = v->n_head_kv;
    // record workgroups: about two per CU over all KV heads; row workgroups: two chunks each
    const int rec_target = 512 / H;
    a.rec_per_wg = a.body_chunks ? (a.body_chunks + rec_target - 1) / rec_target : 1;
    a.n_rec_wg = a.body_chunks ? (a.body_chunks + a.rec_per_wg - 1) / a.rec_per_wg : 0;
    a.row_per_wg = 1;
    const uint32_t tail_pos = a.pend > a.body_end ? a.pend - a.body_end : 0;
    a.n_row_wg = (int) ((a.sink_end + RW_SPAN - 1) / RW_SPAN + (tail_pos + RW_SPAN - 1) / RW_SPAN);
    a.n_wg = a.n_row_wg + a.n_rec_wg;
    if (a.n_wg == 0) { a.n_row_wg = 1; a.n_wg = 1; }    // nothing visible: one empty partial per head
    if (a.n_wg > A2_CMB_MAX) return SJK_ERR_UNSUPPORTED;
    const size_t need = (size_t) H * a.n_wg * A2_Q * (A2_D + 2) * sizeof(float);
    if (need > g_part2_bytes) {
        if (g_part2) (void) hipFree(g_part2);
        g_part2 = nullptr; g_part2_bytes = 0;
        if (hipMalloc((void **) &g_part2, need) != hipSuccess) return SJK_ERR_DEVICE;
        g_part2_bytes = need;
    }
    a.part = g_part2;
    hipStream_t st = (hipStream_t) stream;
    if (a.n_row_wg) hipLaunchKernelGGL(attend2_rows_kernel, dim3((unsigned) a.n_row_wg, (unsigned) H), dim3(64), 0, st, a);
    if (a.n_rec_wg) hipLaunchKernelGGL(attend2_records_kernel, dim3((unsigned) a.n_rec_wg, (unsigned) H), dim3(A2_NT), 0, st, a);
    hipLaunchKernelGGL(attend_combine2, dim3(A2_Q, (unsigned) H, A2_D / 64), dim3(64), 0, st, a);
    return SJK_CHECK_LAUNCH();
}
