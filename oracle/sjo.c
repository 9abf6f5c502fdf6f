/* sjo.c - CPU oracle for the SJ-KVaRN codec hot path (TEST INFRASTRUCTURE ONLY; see sjo.h).
 *
 * Restates the observable behaviour of the reference sj_kvarn.h. Where the stored bytes depend on
 * the order and rounding of arithmetic, the same order is kept (that order IS the format); the
 * code is organised independently. Build: -std=c99 -O2 -ffp-contract=off, no -ffast-math.
 */

#include "sjo.h"
#include "../include/sjk_tables.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------ */
/* bits helpers                                                                                     */
/* ------------------------------------------------------------------------------------------------ */

static float f_of(uint32_t w) { float f; memcpy(&f, &w, 4); return f; }
static uint32_t b_of(float f) { uint32_t w; memcpy(&w, &f, 4); return w; }

static float tq6_cent(int i) { return f_of(SJK_TQ6_CENTROID_BITS[i]); }
static float tq6_mid(int i) { return f_of(SJK_TQ6_MIDPOINT_BITS[i]); }

static const uint16_t *codebook(int bits, int is_v) {
    /* sj_kvarn.h:625-631: 3-bit or 2-bit table, K or V */
    if (bits == 3) return is_v ? SJK_CB3_V : SJK_CB3_K;
    return is_v ? SJK_CB2_V : SJK_CB2_K;
}

/* ternary min/max with the reference's NaN and signed-zero behaviour (sj_kvarn.h:679-682) */
static float fmin_t(float a, float b) { return b < a ? b : a; }
static float fmax_t(float a, float b) { return a < b ? b : a; }
static double dmin_t(double a, double b) { return b < a ? b : a; }
static double dmax_t(double a, double b) { return a < b ? b : a; }

/* ------------------------------------------------------------------------------------------------ */
/* fp16 (sj_kvarn.h:693-731)                                                                        */
/* ------------------------------------------------------------------------------------------------ */

/* Round-to-nearest-even float -> half by integer arithmetic. Matches the reference's bit results
 * for every one of the 2^32 inputs (checked exhaustively against oracle/_ref): NaN -> sign|0x7E00,
 * |f| >= 65520 -> inf, half subnormals rounded on the integer significand. */
uint16_t sjo_f32_to_f16(float f) {
    const uint32_t w = b_of(f), sign = (w >> 16) & 0x8000u, a = w & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t) (sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t) (sign | 0x7C00u);
    if (a >= 0x38800000u) {
        const uint32_t r = a + 0x0FFFu + ((a >> 13) & 1u);
        return (uint16_t) (sign | ((r - 0x38000000u) >> 13));
    } else {
        const uint32_t e = a >> 23;
        uint32_t m, sh, q, rem, half;
        if (e < 102u) return (uint16_t) sign;
        m = (a & 0x7FFFFFu) | 0x800000u;
        sh = 126u - e;
        q = m >> sh;
        rem = m & ((1u << sh) - 1u);
        half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t) (sign | q);
    }
}

float sjo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 31u) return f_of(sign | 0x7F800000u | (m << 13));
    if (e != 0u) return f_of(sign | ((e + 112u) << 23) | (m << 13));
    {
        const float v = (float) m * 0x1p-24f; /* exact: m < 2^10 */
        return sign ? -v : v;
    }
}

static float get_half(const uint8_t *rec, uint32_t off) {
    return sjo_f16_to_f32((uint16_t) (rec[off] | (rec[off + 1] << 8)));
}
static void put_half(uint8_t *rec, uint32_t off, float v) {
    const uint16_t h = sjo_f32_to_f16(v);
    rec[off] = (uint8_t) h;
    rec[off + 1] = (uint8_t) (h >> 8);
}

/* ------------------------------------------------------------------------------------------------ */
/* rotation (sj_kvarn.h:735-759): Sylvester FWHT with stages h = 1, 2, 4, ..., then x * (1/sqrt n)  */
/* ------------------------------------------------------------------------------------------------ */

void sjo_hadamard(float *x, int n) {
    int h, base, j;
    float s;
    for (h = 1; h < n; h *= 2) {
        for (base = 0; base < n; base += 2 * h) {
            for (j = base; j < base + h; ++j) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
        }
    }
    s = 1.0f / sqrtf((float) n);
    for (j = 0; j < n; ++j) x[j] = x[j] * s;
}

void sjo_rotate_heads(float *x, int n_heads, int head_dim) {
    int h;
    for (h = 0; h < n_heads; ++h) sjo_hadamard(x + (size_t) h * head_dim, head_dim);
}

/* ------------------------------------------------------------------------------------------------ */
/* layout and payload order (sj_kvarn.h:763-900)                                                    */
/* ------------------------------------------------------------------------------------------------ */

int sjo_body_resolve(int body, int bits_k, int bits_v) {
    if (body != SJO_BODY_AUTO) return body;
    if ((bits_k == 2 || bits_k == 3) && (bits_v == 2 || bits_v == 3) && bits_v <= bits_k) return SJO_BODY_TRELLIS;
    return SJO_BODY_SCALAR;
}

int sjo_layout_init(sjo_layout *l, int D, int G, int bits_k, int bits_v, int body) {
    uint32_t off;
    if (D < 32 || (D & (D - 1)) || G <= 0 || G % 16) return -1;
    if (bits_k < 2 || bits_k > 4 || bits_v < 2 || bits_v > 4) return -2;
    if (body != SJO_BODY_SCALAR && body != SJO_BODY_TRELLIS) return -3;
    if (body == SJO_BODY_TRELLIS &&
        (bits_k == 4 || bits_v == 4 || bits_v > bits_k || G != SJO_TSEQ || D % SJO_TSEQ)) return -4;
    l->D = D; l->G = G; l->bits_k = bits_k; l->bits_v = bits_v; l->body = body;
    off = 0;
    l->k_payload = off; off += (uint32_t) (D * bits_k / 8) * (uint32_t) G;
    l->v_payload = off; off += (uint32_t) (D * bits_v / 8) * (uint32_t) G;
    l->k_scale = off;   off += 2u * (uint32_t) D;
    l->k_zero = off;    off += 2u * (uint32_t) D;
    l->k_tok = off;     off += 2u * (uint32_t) G;
    l->v_ch = off;      off += 2u * (uint32_t) D;
    l->v_scale = off;   off += 2u * (uint32_t) G;
    l->v_zero = off;    off += 2u * (uint32_t) G;
    l->bytes = off;
    return 0;
}

size_t sjo_record_bytes(int D, int G, int bits_k, int bits_v) {
    return (size_t) G * D * bits_k / 8 + (size_t) G * D * bits_v / 8 + 6 * (size_t) D + 6 * (size_t) G;
}

/* 4-bit scalar sides use the 16x16 fragment order (sj_kvarn.h:803-805) */
static int frag_side(const sjo_layout *l, int bits) {
    return l->body == SJO_BODY_SCALAR && bits == 4 && l->D % 16 == 0 && l->G % 16 == 0;
}

uint32_t sjo_code_bit(const sjo_layout *l, int t, int d, int is_v) {
    const int bits = is_v ? l->bits_v : l->bits_k;
    if (l->body == SJO_BODY_TRELLIS) return ((uint32_t) d * (uint32_t) l->G + (uint32_t) t) * (uint32_t) bits;
    if (!frag_side(l, bits)) return ((uint32_t) t * (uint32_t) l->D + (uint32_t) d) * (uint32_t) bits;
    {
        /* tile (t/16, d/16) is 32 words; within it, one axis picks the word and the other the nibble
         * (sj_kvarn.h:818-832). For V the roles of token and channel are exchanged. */
        const int a = is_v ? d : t, b = is_v ? t : d; /* a: word-row axis, b: nibble axis */
        const int aa = a & 15, bb = b & 15;
        const uint32_t tile = (uint32_t) ((t >> 4) * (l->D / 16) + (d >> 4));
        const uint32_t word = tile * 32u + (uint32_t) (4 * (aa & 7) + ((bb >> 1) & 3));
        const uint32_t nib = (uint32_t) ((aa >> 3) + 2 * (bb >> 3) + 4 * (bb & 1));
        return word * 32u + nib * 4u;
    }
}

int sjo_k_ch_idx(const sjo_layout *l, int d) {
    if (!frag_side(l, l->bits_k)) return d;
    {
        const int c = d >> 4, dd = d & 15, jj = dd >> 1;
        return (jj & 3) * (l->D / 4) + c * 4 + (jj >> 2) * 2 + (dd & 1);
    }
}

int sjo_v_ch_idx(const sjo_layout *l, int d) {
    if (!frag_side(l, l->bits_v)) return d;
    return (d & 7) * (l->D / 8) + (d >> 4) * 2 + ((d >> 3) & 1);
}

static void put_code(uint8_t *p, uint32_t bit, int bits, uint32_t v) {
    const uint32_t sh = bit & 7u, w = (v & ((1u << bits) - 1u)) << sh;
    p[bit >> 3] |= (uint8_t) w;
    if (sh + (uint32_t) bits > 8u) p[(bit >> 3) + 1] |= (uint8_t) (w >> 8);
}

static uint32_t get_code(const uint8_t *p, uint32_t bit, int bits) {
    const uint32_t sh = bit & 7u;
    uint32_t w = p[bit >> 3];
    if (sh + (uint32_t) bits > 8u) w |= (uint32_t) p[(bit >> 3) + 1] << 8;
    return (w >> sh) & ((1u << bits) - 1u);
}

/* codebook index of the code at (channel seq, token i) of a channel-major trellis stream: the code
 * over the 6 preceding stream bits of the same channel, zeros before the channel start
 * (sj_kvarn.h:882-900) */
static uint32_t trellis_window(const uint8_t *payload, int bits, int seq, int i) {
    const uint32_t bit = ((uint32_t) seq * SJO_TSEQ + (uint32_t) i) * (uint32_t) bits;
    const int need = (SJO_THIST + bits - 1) / bits; /* codes of history that fit in 6 bits */
    uint32_t w;
    int k;
    if (i >= need) {
        /* all 6 history bits lie inside this channel's stream: read them with the code */
        const uint32_t start = bit - SJO_THIST;
        const uint32_t v = (uint32_t) payload[start >> 3] | ((uint32_t) payload[(start >> 3) + 1] << 8);
        return (v >> (start & 7u)) & ((1u << (SJO_THIST + bits)) - 1u);
    }
    w = get_code(payload, bit, bits) << SJO_THIST;
    for (k = 1; k <= i; ++k) w |= get_code(payload, bit - (uint32_t) (k * bits), bits) << (SJO_THIST - k * bits);
    return w;
}

/* ------------------------------------------------------------------------------------------------ */
/* seal (sj_kvarn.h:906-1174)                                                                        */
/* ------------------------------------------------------------------------------------------------ */

typedef struct {
    float *tile, *bal, *srow, *scol, *qlo, *qstep, *y, *cbf, *M, *Mn;
    double *lrow, *lcol;
    uint8_t *codes, *arg;
} seal_ws;

static size_t round8(size_t x) { return (x + 7u) & ~(size_t) 7u; }

/* scratch carve; the total equals sj_kvarn_seal_workspace_bytes (sj_kvarn.h:912-937) */
static size_t ws_carve(const sjo_layout *l, void *base, seal_ws *w) {
    const size_t DG = (size_t) l->D * (size_t) l->G, R = (size_t) (l->D > l->G ? l->D : l->G);
    const size_t sizes[14] = {
        4 * DG, 4 * DG, 4 * R, 4 * R, 4 * R, 4 * R, 8 * R, 8 * R, 4 * SJO_TSEQ, 4 * 512,
        4 * SJO_NSTATE, 4 * SJO_NSTATE, SJO_TSEQ, (size_t) SJO_TSEQ * SJO_NSTATE };
    size_t off[14], at = 0;
    int i;
    for (i = 0; i < 14; ++i) { off[i] = at; at = round8(at + sizes[i]); }
    if (w) {
        uint8_t *p = (uint8_t *) base;
        w->tile = (float *) (p + off[0]);   w->bal = (float *) (p + off[1]);
        w->srow = (float *) (p + off[2]);   w->scol = (float *) (p + off[3]);
        w->qlo = (float *) (p + off[4]);    w->qstep = (float *) (p + off[5]);
        w->lrow = (double *) (p + off[6]);  w->lcol = (double *) (p + off[7]);
        w->y = (float *) (p + off[8]);      w->cbf = (float *) (p + off[9]);
        w->M = (float *) (p + off[10]);     w->Mn = (float *) (p + off[11]);
        w->codes = p + off[12];             w->arg = p + off[13];
    }
    return at;
}

size_t sjo_seal_workspace_bytes(const sjo_layout *l) { return ws_carve(l, NULL, NULL); }

/* ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7)) (sj_kvarn.h:943-953) */
static double tree8(const double *p) {
    const double a = p[0] + p[1], b = p[2] + p[3], c = p[4] + p[5], d = p[6] + p[7];
    return (a + b) + (c + d);
}

/* sample standard deviation of n strided values: 8 contiguous chunks summed sequentially in double,
 * tree-combined; second moment with fma (sj_kvarn.h:956-978) */
static float chunked_std(const float *x, int n, size_t stride) {
    const int len = n / 8;
    double part[8], mean, m2;
    int c, i;
    for (c = 0; c < 8; ++c) {
        double s = 0.0;
        for (i = 0; i < len; ++i) s = s + (double) x[(size_t) (c * len + i) * stride];
        part[c] = s;
    }
    mean = tree8(part) / (double) n;
    for (c = 0; c < 8; ++c) {
        double s = 0.0;
        for (i = 0; i < len; ++i) {
            const double d = (double) x[(size_t) (c * len + i) * stride] - mean;
            s = fma(d, d, s);
        }
        part[c] = s;
    }
    m2 = tree8(part);
    return (float) sqrt(m2 / (double) (n > 1 ? n - 1 : 1));
}

/* cur = (M / s_col) / s_row, two correctly rounded divisions (sj_kvarn.h:980-987) */
static void rebalance(const float *M, int R, int C, const float *srow, const float *scol, float *cur) {
    int r, c;
    for (r = 0; r < R; ++r)
        for (c = 0; c < C; ++c) cur[(size_t) r * C + c] = (M[(size_t) r * C + c] / scol[c]) / srow[r];
}

/* one log-domain scale update: clamp the std, accumulate its log, clamp, exponentiate
 * (sj_kvarn.h:1000-1002, 1006-1008) */
static float log_step(double *acc, float sd) {
    const float s = fmin_t(fmax_t(sd, 1e-3f), 1e3f);
    *acc = dmin_t(dmax_t(*acc + log((double) s), -0.3), 10.0);
    return (float) exp(*acc);
}

/* log_step over arrays: acc[i] is updated in place, scale[i] = the returned scale (the checker of the
 * device's log / exp in the balance, whose results the golden vectors pin through the seal) */
void sjo_balance_step(const float *sd, double *acc, float *scale, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) scale[i] = log_step(&acc[i], sd[i]);
}

/* exactly `iters` column-then-row passes over the row-major [R][C] tile (sj_kvarn.h:992-1012) */
static void variance_balance(const float *M, int R, int C, int iters, float *srow, float *scol, float *cur,
                             double *lrow, double *lcol) {
    int it, r, c;
    for (c = 0; c < C; ++c) { scol[c] = 1.0f; lcol[c] = 0.0; }
    for (r = 0; r < R; ++r) { srow[r] = 1.0f; lrow[r] = 0.0; }
    rebalance(M, R, C, srow, scol, cur);
    for (it = 0; it < iters; ++it) {
        for (c = 0; c < C; ++c) scol[c] = log_step(&lcol[c], chunked_std(cur + c, R, (size_t) C));
        rebalance(M, R, C, srow, scol, cur);
        for (r = 0; r < R; ++r) srow[r] = log_step(&lrow[r], chunked_std(cur + (size_t) r * C, C, 1));
        rebalance(M, R, C, srow, scol, cur);
    }
}

/* code = clamp(rint((x - lo) / step), 0, qmax), ties to even (sj_kvarn.h:1014-1019) */
static uint32_t round_code(float x, float lo, float step, uint32_t qmax) {
    float r = nearbyintf((x - lo) / step);
    if (r < 0.0f) r = 0.0f;
    if (r > (float) qmax) r = (float) qmax;
    return (uint32_t) r;
}

/* Viterbi over one channel: backward DP from the last token, 64 states, branch j of state s reads
 * window s + 64 j and continues in state (s + 64 j) >> bits; cost (y - cb)^2 + M with one rounding
 * per op; strict < over ascending j; traceback from state 0 (sj_kvarn.h:1025-1053) */
static void viterbi(const float *y, int n, int bits, const float *cbf, uint8_t *codes, float *M, float *Mn,
                    uint8_t *arg) {
    const int nb = 1 << bits;
    int i, s, j;
    for (s = 0; s < SJO_NSTATE; ++s) M[s] = 0.0f;
    for (i = n - 1; i >= 0; --i) {
        float *swap;
        for (s = 0; s < SJO_NSTATE; ++s) {
            float best = INFINITY;
            int pick = 0;
            for (j = 0; j < nb; ++j) {
                const int win = s + SJO_NSTATE * j;
                const float d = y[i] - cbf[win];
                const float e = d * d;
                const float cost = e + M[win >> bits];
                if (cost < best) { best = cost; pick = j; }
            }
            Mn[s] = best;
            arg[(size_t) i * SJO_NSTATE + s] = (uint8_t) pick;
        }
        swap = M; M = Mn; Mn = swap;
    }
    s = 0;
    for (i = 0; i < n; ++i) {
        j = arg[(size_t) i * SJO_NSTATE + s];
        codes[i] = (uint8_t) j;
        s = (s + SJO_NSTATE * j) >> bits;
    }
}

/* moment-matching refit of each row's affine after trellis coding (sj_kvarn.h:1078-1109) */
static void trellis_refit(const sjo_layout *l, const float *bal, int R, int C, const float *srow, int is_v,
                          const uint8_t *payload, uint8_t *rec) {
    const int bits = is_v ? l->bits_v : l->bits_k;
    const uint16_t *cb = codebook(bits, is_v);
    int r, c;
    for (r = 0; r < R; ++r) {
        double sx = 0.0, sy = 0.0, sxx = 0.0, syy = 0.0, vx, vy, a, b;
        const double n = (double) C;
        for (c = 0; c < C; ++c) {
            const int tok = is_v ? r : c, ch = is_v ? c : r;
            const double x = (double) bal[(size_t) r * C + c];
            const double yh = (double) sjo_f16_to_f32(cb[trellis_window(payload, bits, ch, tok)]);
            sx = sx + x;
            sy = sy + yh;
            sxx = sxx + x * x;
            syy = syy + yh * yh;
        }
        vy = n * syy - sy * sy;
        if (!(vy > 0.0)) continue;
        vx = n * sxx - sx * sx;
        if (!(vx > 0.0)) continue;
        a = sqrt(vx / vy);
        b = (sx - a * sy) / n;
        if (!(a > 0.0) || b != b || a > 1e30 || fabs(b) > 1e30) continue;
        {
            const uint32_t ri = (uint32_t) (is_v ? r : sjo_k_ch_idx(l, r));
            put_half(rec, (is_v ? l->v_scale : l->k_scale) + 2u * ri, srow[r] * (float) a);
            put_half(rec, (is_v ? l->v_zero : l->k_zero) + 2u * ri, srow[r] * (float) b);
        }
    }
}

/* quantize one balanced side; K: rows = channels [D][G], V: rows = tokens [G][D]
 * (sj_kvarn.h:1112-1147) */
static void quantize_side(const sjo_layout *l, int is_v, uint8_t *rec, seal_ws *w) {
    const int D = l->D, G = l->G, R = is_v ? G : D, C = is_v ? D : G;
    const int bits = is_v ? l->bits_v : l->bits_k;
    const uint32_t qmax = (1u << bits) - 1u;
    const int trellis = l->body == SJO_BODY_TRELLIS;
    uint8_t *payload = rec + (is_v ? l->v_payload : l->k_payload);
    int r, c;
    for (r = 0; r < R; ++r) {
        const float *row = w->bal + (size_t) r * C;
        float lo = row[0], hi = row[0], step;
        uint32_t ri;
        for (c = 1; c < C; ++c) { lo = fmin_t(lo, row[c]); hi = fmax_t(hi, row[c]); }
        step = fmax_t((hi - lo) / (float) qmax, 1e-10f);
        ri = (uint32_t) (is_v ? r : sjo_k_ch_idx(l, r));
        put_half(rec, (is_v ? l->v_scale : l->k_scale) + 2u * ri, w->srow[r] * step);
        put_half(rec, (is_v ? l->v_zero : l->k_zero) + 2u * ri, w->srow[r] * lo);
        if (trellis) { w->qlo[r] = lo; w->qstep[r] = step; continue; }
        for (c = 0; c < C; ++c) {
            const int t = is_v ? r : c, d = is_v ? c : r;
            put_code(payload, sjo_code_bit(l, t, d, is_v), bits, round_code(row[c], lo, step, qmax));
        }
    }
    if (trellis) {
        /* one Viterbi sequence per channel along the G tokens (sj_kvarn.h:1057-1073) */
        const uint16_t *cb = codebook(bits, is_v);
        const int nwin = 1 << (SJO_THIST + bits);
        int d, t;
        for (d = 0; d < nwin; ++d) w->cbf[d] = sjo_f16_to_f32(cb[d]);
        for (d = 0; d < D; ++d) {
            for (t = 0; t < G; ++t) {
                const int rr = is_v ? t : d, cc = is_v ? d : t;
                w->y[t] = (w->bal[(size_t) rr * C + cc] - w->qlo[rr]) / w->qstep[rr];
            }
            viterbi(w->y, G, bits, w->cbf, w->codes, w->M, w->Mn, w->arg);
            for (t = 0; t < G; ++t)
                put_code(payload, ((uint32_t) d * (uint32_t) G + (uint32_t) t) * (uint32_t) bits, bits, w->codes[t]);
        }
        trellis_refit(l, w->bal, R, C, w->srow, is_v, payload, rec);
    }
    /* column scales absorbed into the record: Ktok[t], Vch[v_ch_idx(d)] */
    for (c = 0; c < C; ++c) {
        const uint32_t off = is_v ? l->v_ch + 2u * (uint32_t) sjo_v_ch_idx(l, c) : l->k_tok + 2u * (uint32_t) c;
        put_half(rec, off, w->scol[c]);
    }
}

void sjo_seal_group(const sjo_layout *l, const uint16_t *K, const uint16_t *V, size_t row_stride, int iters,
                    uint8_t *rec, void *work) {
    const int D = l->D, G = l->G;
    seal_ws w;
    int t, d;
    ws_carve(l, work, &w);
    memset(rec, 0, l->bytes);
    /* K tile [D][G]: rows are channels */
    for (t = 0; t < G; ++t)
        for (d = 0; d < D; ++d) w.tile[(size_t) d * G + t] = sjo_f16_to_f32(K[(size_t) t * row_stride + d]);
    variance_balance(w.tile, D, G, iters, w.srow, w.scol, w.bal, w.lrow, w.lcol);
    quantize_side(l, 0, rec, &w);
    /* V tile [G][D]: rows are tokens */
    for (t = 0; t < G; ++t)
        for (d = 0; d < D; ++d) w.tile[(size_t) t * D + d] = sjo_f16_to_f32(V[(size_t) t * row_stride + d]);
    variance_balance(w.tile, G, D, iters, w.srow, w.scol, w.bal, w.lrow, w.lcol);
    quantize_side(l, 1, rec, &w);
}

/* ------------------------------------------------------------------------------------------------ */
/* decode (sj_kvarn.h:1178-1207)                                                                     */
/* ------------------------------------------------------------------------------------------------ */

static float code_value(const sjo_layout *l, const uint8_t *rec, int t, int d, int is_v) {
    const int bits = is_v ? l->bits_v : l->bits_k;
    const uint8_t *payload = rec + (is_v ? l->v_payload : l->k_payload);
    if (l->body == SJO_BODY_TRELLIS) return sjo_f16_to_f32(codebook(bits, is_v)[trellis_window(payload, bits, d, t)]);
    return (float) get_code(payload, sjo_code_bit(l, t, d, is_v), bits);
}

void sjo_decode_k_row(const sjo_layout *l, const uint8_t *rec, int t, float *out) {
    const float tok = get_half(rec, l->k_tok + 2u * (uint32_t) t);
    int d;
    for (d = 0; d < l->D; ++d) {
        const uint32_t ci = (uint32_t) sjo_k_ch_idx(l, d);
        const float q = code_value(l, rec, t, d, 0);
        out[d] = (q * get_half(rec, l->k_scale + 2u * ci) + get_half(rec, l->k_zero + 2u * ci)) * tok;
    }
}

void sjo_decode_v_row(const sjo_layout *l, const uint8_t *rec, int t, float *out) {
    const float sc = get_half(rec, l->v_scale + 2u * (uint32_t) t), zp = get_half(rec, l->v_zero + 2u * (uint32_t) t);
    int d;
    for (d = 0; d < l->D; ++d) {
        const float q = code_value(l, rec, t, d, 1);
        out[d] = (q * sc + zp) * get_half(rec, l->v_ch + 2u * (uint32_t) sjo_v_ch_idx(l, d));
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* staging (sj_kvarn.h:1211-1284)                                                                    */
/* ------------------------------------------------------------------------------------------------ */

/* level index = number of midpoints m with !(v < mid[m]); equals the reference's binary search
 * over the sorted midpoints for every v, NaN included (-> 63) (sj_kvarn.h:1211-1219) */
static int tq6_level(float v) {
    int m, k = 0;
    for (m = 0; m < 63; ++m) k += !(v < tq6_mid(m));
    return k;
}

void sjo_tq6_quantize_row(const float *x, uint8_t *blocks, int n) {
    int b, i;
    for (b = 0; b < n / SJO_QK; ++b) {
        const float *src = x + (size_t) b * SJO_QK;
        uint8_t *blk = blocks + (size_t) b * SJO_TQ6_BYTES;
        uint8_t code[SJO_QK];
        float nsq = 0.0f, norm, inv = 0.0f, csq = 0.0f, cn, scale;
        uint16_t h;
        for (i = 0; i < SJO_QK; ++i) nsq = nsq + src[i] * src[i];
        norm = sqrtf(nsq);
        if (norm > 1e-10f) inv = 1.0f / norm;
        for (i = 0; i < SJO_QK; ++i) code[i] = (uint8_t) tq6_level(norm > 1e-10f ? src[i] * inv : 0.0f);
        for (i = 0; i < SJO_QK; ++i) csq = csq + tq6_cent(code[i]) * tq6_cent(code[i]);
        cn = sqrtf(csq);
        scale = cn > 1e-10f ? norm / cn : norm;
        h = sjo_f32_to_f16(scale);
        memset(blk, 0, SJO_TQ6_BYTES);
        blk[0] = (uint8_t) h;
        blk[1] = (uint8_t) (h >> 8);
        for (i = 0; i < SJO_QK; ++i) {
            blk[2 + i / 2] |= (uint8_t) ((code[i] & 15u) << (4 * (i & 1)));
            blk[66 + i / 4] |= (uint8_t) (((code[i] >> 4) & 3u) << (2 * (i & 3)));
        }
    }
}

void sjo_tq6_dequantize_row(const uint8_t *blocks, float *x, int n) {
    int b, i;
    for (b = 0; b < n / SJO_QK; ++b) {
        const uint8_t *blk = blocks + (size_t) b * SJO_TQ6_BYTES;
        const float norm = sjo_f16_to_f32((uint16_t) (blk[0] | (blk[1] << 8)));
        for (i = 0; i < SJO_QK; ++i) {
            const int code = ((blk[2 + i / 2] >> (4 * (i & 1))) & 15) | (((blk[66 + i / 4] >> (2 * (i & 3))) & 3) << 4);
            x[(size_t) b * SJO_QK + i] = tq6_cent(code) * norm;
        }
    }
}

size_t sjo_stage_row_bytes(int staging, int D) {
    return staging == SJO_STAGING_F16 ? (size_t) D * 2 : (size_t) (D / SJO_QK) * SJO_TQ6_BYTES;
}

void sjo_stage_row(int staging, const float *x_rot, void *dst, int D) {
    if (staging == SJO_STAGING_F16) {
        uint8_t *o = (uint8_t *) dst;
        int i;
        for (i = 0; i < D; ++i) {
            const uint16_t h = sjo_f32_to_f16(x_rot[i]);
            o[2 * i] = (uint8_t) h;
            o[2 * i + 1] = (uint8_t) (h >> 8);
        }
        return;
    }
    sjo_tq6_quantize_row(x_rot, (uint8_t *) dst, D);
}

void sjo_unstage_row(int staging, const void *src, float *x_rot, int D) {
    if (staging == SJO_STAGING_F16) {
        const uint8_t *p = (const uint8_t *) src;
        int i;
        for (i = 0; i < D; ++i) x_rot[i] = sjo_f16_to_f32((uint16_t) (p[2 * i] | (p[2 * i + 1] << 8)));
        return;
    }
    sjo_tq6_dequantize_row((const uint8_t *) src, x_rot, D);
}

/* ------------------------------------------------------------------------------------------------ */
/* attention helpers (sj_kvarn.h:1288-1311)                                                          */
/* ------------------------------------------------------------------------------------------------ */

static float seq_dot(const float *a, const float *b, int n) {
    float s = 0.0f;
    int i;
    for (i = 0; i < n; ++i) s = s + a[i] * b[i];
    return s;
}

void sjo_record_scores(const sjo_layout *l, const uint8_t *rec, const float *q, int n, float *scores) {
    float row[1024];
    int t;
    for (t = 0; t < n; ++t) { sjo_decode_k_row(l, rec, t, row); scores[t] = seq_dot(q, row, l->D); }
}

void sjo_record_accum_v(const sjo_layout *l, const uint8_t *rec, const float *w, int n, float *acc) {
    float row[1024];
    int t, d;
    for (t = 0; t < n; ++t) {
        sjo_decode_v_row(l, rec, t, row);
        for (d = 0; d < l->D; ++d) acc[d] = acc[d] + w[t] * row[d];
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* journal policy (sj_kvarn.h:1315-1407)                                                             */
/* ------------------------------------------------------------------------------------------------ */

void sjo_policy_init(sjo_policy *p, uint32_t sink, uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t flush_chunk) {
    p->sink = sink; p->tail = tail; p->tail_max = tail_max; p->group = group; p->flush_chunk = flush_chunk;
    sjo_policy_reset(p);
}

void sjo_policy_reset(sjo_policy *p) {
    p->B = p->B_prev = p->B_pending = p->sink;
    p->draining = 0;
}

uint32_t sjo_policy_begin_ubatch(sjo_policy *p, uint32_t pos0, uint32_t n_tokens) {
    const int due = p->tail_max == 0 || p->draining || (pos0 > p->B && pos0 - p->B >= p->tail_max);
    p->B_pending = p->B;
    p->draining = 0;
    if (due && pos0 > p->sink + p->tail) {
        uint32_t target = sjo_group_floor(p->sink, p->group, pos0 - p->tail);
        if (target < p->B) target = p->B;
        if (p->tail_max > 0 && p->flush_chunk > 0 && n_tokens < p->group && target > p->B + p->group * p->flush_chunk) {
            target = p->B + p->group * p->flush_chunk;
            p->draining = 1;
        }
        p->B_pending = target;
    }
    return p->B_pending;
}

void sjo_policy_commit(sjo_policy *p) { p->B_prev = p->B; p->B = p->B_pending; }

uint32_t sjo_policy_idle(sjo_policy *p, uint32_t end, uint32_t keep_recent) {
    uint32_t target;
    int clamped = 0;
    p->B_pending = p->B;
    if (p->tail_max == 0 || end <= p->sink + p->tail) return p->B;
    target = sjo_group_floor(p->sink, p->group, end - p->tail);
    if (keep_recent > p->tail) {
        const uint32_t from = end > keep_recent ? end - keep_recent : 0;
        const uint32_t lim = from <= p->sink ? p->sink : sjo_group_floor(p->sink, p->group, from);
        if (lim < target) { target = lim; clamped = 1; }
    }
    if (!clamped) p->draining = 0;
    if (target <= p->B) return p->B;
    p->B_pending = target;
    return target;
}

uint32_t sjo_group_floor(uint32_t sink, uint32_t group, uint32_t pos) {
    return pos <= sink ? pos : sink + group * ((pos - sink) / group);
}

uint32_t sjo_policy_trunc_floor(const sjo_policy *p, uint32_t pos) {
    return (pos >= p->B || pos <= p->sink) ? pos : sjo_group_floor(p->sink, p->group, pos);
}

uint32_t sjo_policy_truncate(sjo_policy *p, uint32_t pos, uint32_t *n_dropped) {
    uint32_t r;
    if (n_dropped) *n_dropped = 0;
    if (p->B_pending != p->B) return SJO_NO_POS;
    r = sjo_policy_trunc_floor(p, pos);
    if (r < p->B) {
        const uint32_t nb = r > p->sink ? r : p->sink;
        if (n_dropped) *n_dropped = (p->B - nb) / p->group;
        p->B = p->B_prev = p->B_pending = nb;
        p->draining = 0;
    }
    return r;
}

uint32_t sjo_ring_capacity(uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t n_ubatch) {
    const uint32_t need = (tail > tail_max ? tail : tail_max) + group + 2u * n_ubatch;
    return (need + 127u) / 128u * 128u;
}

uint32_t sjo_ring_slot(uint32_t sink, uint32_t cap, uint32_t pos) { return (pos - sink) % cap; }

/* ------------------------------------------------------------------------------------------------ */
/* per-layer cache (sj_kvarn.h:1411-1603)                                                            */
/* ------------------------------------------------------------------------------------------------ */

void sjo_config_default_into(sjo_config *c, int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch) {
    c->head_dim = head_dim; c->n_head_kv = n_head_kv; c->group = 128; c->bits_k = 4; c->bits_v = 4;
    c->body = SJO_BODY_AUTO; c->iters = 16; c->staging = SJO_STAGING_TQ6; c->sink_type = SJO_SINK_F16;
    c->sink = 128; c->tail = 4096; c->tail_max = 8192; c->flush_chunk = 0; c->n_ubatch = n_ubatch; c->n_ctx = n_ctx;
}

sjo_config sjo_config_default(int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch) {
    sjo_config c;
    sjo_config_default_into(&c, head_dim, n_head_kv, n_ctx, n_ubatch);
    return c;
}

uint8_t *sjo_layer_record(const sjo_layer *L, uint32_t g, int h) {
    const uint32_t blk = L->blocks ? L->blocks[g] : g;
    return L->body + ((size_t) blk * (size_t) L->cfg.n_head_kv + (size_t) h) * L->lay.bytes;
}

static size_t sink_entry_bytes(const sjo_layer *L) {
    return L->cfg.sink_type == SJO_SINK_F16 ? (size_t) L->cfg.head_dim * 4 : 2 * L->stage_bytes;
}
static uint8_t *sink_entry(const sjo_layer *L, uint32_t pos, int h) {
    return L->sink + ((size_t) pos * (size_t) L->cfg.n_head_kv + (size_t) h) * sink_entry_bytes(L);
}
static uint8_t *ring_entry(const sjo_layer *L, uint32_t pos, int h) {
    return L->ring + ((size_t) sjo_ring_slot(L->cfg.sink, L->cap, pos) * (size_t) L->cfg.n_head_kv + (size_t) h) *
                         2 * L->stage_bytes;
}

static int layer_setup(sjo_layer *L, const sjo_config *cfg, int own_body) {
    const int D = cfg->head_dim, H = cfg->n_head_kv;
    int rc;
    memset(L, 0, sizeof(*L));
    L->cfg = *cfg;
    L->cfg.body = sjo_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (D % SJO_QK || cfg->group % 16 || cfg->sink == 0 || cfg->sink % 64 || cfg->tail % (uint32_t) cfg->group ||
        (cfg->tail_max != 0 && (cfg->tail_max < cfg->tail || cfg->tail_max % 128))) return -10;
    rc = sjo_layout_init(&L->lay, D, cfg->group, cfg->bits_k, cfg->bits_v, L->cfg.body);
    if (rc) return rc;
    L->cap = sjo_ring_capacity(cfg->tail, cfg->tail_max, (uint32_t) cfg->group, cfg->n_ubatch);
    L->n_groups = cfg->n_ctx > cfg->sink ? (cfg->n_ctx - cfg->sink + (uint32_t) cfg->group - 1) / (uint32_t) cfg->group : 1;
    L->stage_bytes = sjo_stage_row_bytes(cfg->staging, D);
    L->ring = (uint8_t *) calloc((size_t) L->cap * H, 2 * L->stage_bytes);
    L->sink = (uint8_t *) calloc((size_t) cfg->sink * H, cfg->sink_type == SJO_SINK_F16 ? (size_t) D * 4 : 2 * L->stage_bytes);
    L->owns_body = own_body;
    L->body = own_body ? (uint8_t *) calloc((size_t) L->n_groups * H, L->lay.bytes) : NULL;
    L->work = malloc(sjo_seal_workspace_bytes(&L->lay));
    L->kstage = (uint16_t *) malloc((size_t) cfg->group * D * 2);
    L->vstage = (uint16_t *) malloc((size_t) cfg->group * D * 2);
    if (!L->ring || !L->sink || (own_body && !L->body) || !L->work || !L->kstage || !L->vstage) {
        sjo_layer_free(L);
        return -11;
    }
    return 0;
}

int sjo_layer_init(sjo_layer *L, const sjo_config *cfg) { return layer_setup(L, cfg, 1); }

void sjo_layer_free(sjo_layer *L) {
    free(L->ring); free(L->sink); if (L->owns_body) free(L->body); free(L->work); free(L->kstage); free(L->vstage);
    L->ring = L->sink = L->body = NULL; L->blocks = NULL; L->owns_body = 0; L->work = NULL; L->kstage = L->vstage = NULL;
}

void sjo_layer_store(sjo_layer *L, uint32_t pos, const float *k_rot, const float *v_rot) {
    const int D = L->cfg.head_dim, H = L->cfg.n_head_kv;
    int h, i;
    for (h = 0; h < H; ++h) {
        const float *kr = k_rot + (size_t) h * D, *vr = v_rot + (size_t) h * D;
        if (pos < L->cfg.sink && L->cfg.sink_type == SJO_SINK_F16) {
            uint8_t *e = sink_entry(L, pos, h);
            for (i = 0; i < D; ++i) {
                const uint16_t a = sjo_f32_to_f16(kr[i]), b = sjo_f32_to_f16(vr[i]);
                e[2 * i] = (uint8_t) a; e[2 * i + 1] = (uint8_t) (a >> 8);
                e[2 * (D + i)] = (uint8_t) b; e[2 * (D + i) + 1] = (uint8_t) (b >> 8);
            }
        } else {
            uint8_t *e = pos < L->cfg.sink ? sink_entry(L, pos, h) : ring_entry(L, pos, h);
            sjo_stage_row(L->cfg.staging, kr, e, D);
            sjo_stage_row(L->cfg.staging, vr, e + L->stage_bytes, D);
        }
    }
}

/* seal [B_from, B_to): each ring row dequantized, rounded to fp16, sealed (sj_kvarn.h:1494-1514) */
void sjo_layer_seal(sjo_layer *L, uint32_t B_from, uint32_t B_to) {
    const int D = L->cfg.head_dim, H = L->cfg.n_head_kv, G = L->cfg.group;
    float row[1024];
    uint32_t p0;
    int h, t, i;
    for (p0 = B_from; p0 < B_to; p0 += (uint32_t) G) {
        const uint32_t g = (p0 - L->cfg.sink) / (uint32_t) G;
        for (h = 0; h < H; ++h) {
            for (t = 0; t < G; ++t) {
                const uint8_t *e = ring_entry(L, p0 + (uint32_t) t, h);
                sjo_unstage_row(L->cfg.staging, e, row, D);
                for (i = 0; i < D; ++i) L->kstage[(size_t) t * D + i] = sjo_f32_to_f16(row[i]);
                sjo_unstage_row(L->cfg.staging, e + L->stage_bytes, row, D);
                for (i = 0; i < D; ++i) L->vstage[(size_t) t * D + i] = sjo_f32_to_f16(row[i]);
            }
            sjo_seal_group(&L->lay, L->kstage, L->vstage, (size_t) D, L->cfg.iters, sjo_layer_record(L, g, h), L->work);
        }
    }
}

void sjo_layer_kv_row(const sjo_layer *L, uint32_t B, uint32_t pos, int h, float *k, float *v) {
    const int D = L->cfg.head_dim;
    int i;
    if (pos >= L->cfg.sink && pos < B) {
        const uint32_t off = pos - L->cfg.sink, G = (uint32_t) L->cfg.group;
        const uint8_t *rec = sjo_layer_record(L, off / G, h);
        sjo_decode_k_row(&L->lay, rec, (int) (off % G), k);
        sjo_decode_v_row(&L->lay, rec, (int) (off % G), v);
    } else if (pos < L->cfg.sink && L->cfg.sink_type == SJO_SINK_F16) {
        const uint8_t *e = sink_entry(L, pos, h);
        for (i = 0; i < D; ++i) {
            k[i] = sjo_f16_to_f32((uint16_t) (e[2 * i] | (e[2 * i + 1] << 8)));
            v[i] = sjo_f16_to_f32((uint16_t) (e[2 * (D + i)] | (e[2 * (D + i) + 1] << 8)));
        }
    } else {
        const uint8_t *e = pos < L->cfg.sink ? sink_entry(L, pos, h) : ring_entry(L, pos, h);
        sjo_unstage_row(L->cfg.staging, e, k, D);
        sjo_unstage_row(L->cfg.staging, e + L->stage_bytes, v, D);
    }
}

/* causal online softmax over [0, min(N, qpos+1)) in position order (sj_kvarn.h:1535-1564) */
void sjo_layer_attend_row(const sjo_layer *L, uint32_t B, uint32_t N, const float *q_rot, int h, uint32_t qpos,
                          float scale, float *out_rot) {
    const int D = L->cfg.head_dim;
    const uint32_t end = N < qpos + 1 ? N : qpos + 1;
    float krow[1024], vrow[1024], acc[1024], mx = -INFINITY, den = 0.0f, inv;
    uint32_t p;
    int d;
    for (d = 0; d < D; ++d) acc[d] = 0.0f;
    for (p = 0; p < end; ++p) {
        float s, shrink = 1.0f, wv = 1.0f;
        sjo_layer_kv_row(L, B, p, h, krow, vrow);
        s = seq_dot(q_rot, krow, D) * scale;
        if (s > mx) {
            const float old = mx;
            mx = s;
            shrink = expf(old - mx);
            for (d = 0; d < D; ++d) acc[d] = acc[d] * shrink;
        } else {
            wv = expf(s - mx);
        }
        for (d = 0; d < D; ++d) acc[d] = acc[d] + vrow[d] * wv;
        den = den * shrink + wv;
    }
    inv = den == 0.0f ? 0.0f : 1.0f / den;
    for (d = 0; d < D; ++d) out_rot[d] = acc[d] * inv;
}

void sjo_layer_truncate(sjo_layer *L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume) {
    const uint32_t S = L->cfg.sink, G = (uint32_t) L->cfg.group;
    const int H = L->cfg.n_head_kv;
    uint32_t g, pos, from;
    int h;
    if (B_new < B_old) {
        for (g = (B_new - S) / G; g < (B_old - S) / G; ++g) {
            if (L->blocks && L->blocks[g] == SJO_NO_BLOCK) continue;
            for (h = 0; h < H; ++h) memset(sjo_layer_record(L, g, h), 0, L->lay.bytes);
        }
    }
    for (pos = resume; pos < n_old && pos < S; ++pos)
        for (h = 0; h < H; ++h) memset(sink_entry(L, pos, h), 0, sink_entry_bytes(L));
    from = resume > S ? resume : S;
    if (n_old > from && n_old - from > L->cap) from = n_old - L->cap;
    for (pos = from; pos < n_old; ++pos)
        for (h = 0; h < H; ++h) memset(ring_entry(L, pos, h), 0, 2 * L->stage_bytes);
}

const char *sjo_strerror(int code) {
    switch (code) {
    case 0: return "ok";
    case -1: return "layout: head_dim must be a power of two >= 32 and group a multiple of 16";
    case -2: return "layout: bits_k and bits_v must be 2, 3 or 4";
    case -3: return "layout: unknown body type";
    case -4: return "layout: trellis bodies need 3/3, 3/2 or 2/2 bits, group 128 and head_dim a multiple of 128";
    case -10: return "config: head_dim % 128, group % 16, sink (non-zero, % 64), tail % group or tail_max invalid";
    case -11: return "out of memory";
    case -100: return "invalid argument";
    case -101: return "out of memory";
    case -102: return "destination buffer too small for the sequence state";
    case -103: return "state stream is shorter than its header says";
    case -104: return "not an SJ-KVaRN sequence state (bad magic)";
    case -105: return "unsupported SJ-KVaRN state version";
    case -106: return "state was written with a different record/staging byte format";
    case -107: return "state checksum or consistency check failed";
    case -108: return "a seal is pending (call commit first)";
    case -109: return "state does not fit this cache (context, ring or group capacity)";
    case -110: return "record pool has no free block";
    case -120: return "config mismatch: head_dim";
    case -121: return "config mismatch: n_head_kv";
    case -122: return "config mismatch: group size";
    case -123: return "config mismatch: sink length or sink type";
    case -124: return "config mismatch: bits_k/bits_v";
    case -125: return "config mismatch: body type (scalar/trellis)";
    case -126: return "config mismatch: variance-balancing iterations";
    case -127: return "config mismatch: staging type";
    case -128: return "config mismatch: tail, tail_max or flush_chunk";
    case -129: return "config mismatch: rotation";
    case -130: return "config mismatch: trellis codebook";
    case -131: return "config mismatch: number of layers";
    default: return "unknown SJ-KVaRN status code";
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* pool / sequence (sj_kvarn.h:1645-1809)                                                            */
/* ------------------------------------------------------------------------------------------------ */

int sjo_pool_init(sjo_pool *pool, const sjo_config *cfg, int n_layers, uint32_t n_blocks) {
    uint32_t i;
    int rc;
    memset(pool, 0, sizeof(*pool));
    if (n_layers <= 0 || n_blocks == 0 || cfg->n_head_kv <= 0) return -100;
    pool->cfg = *cfg;
    pool->cfg.body = sjo_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    rc = sjo_layout_init(&pool->lay, cfg->head_dim, cfg->group, cfg->bits_k, cfg->bits_v, pool->cfg.body);
    if (rc) return rc;
    pool->n_layers = n_layers;
    pool->n_blocks = n_blocks;
    pool->body = (uint8_t *) calloc((size_t) n_layers * n_blocks * (size_t) cfg->n_head_kv, pool->lay.bytes);
    pool->free_ids = (uint32_t *) malloc((size_t) n_blocks * sizeof(uint32_t));
    if (!pool->body || !pool->free_ids) { sjo_pool_free(pool); return -101; }
    for (i = 0; i < n_blocks; ++i) pool->free_ids[i] = n_blocks - 1u - i; /* LIFO: block 0 first */
    pool->n_free = n_blocks;
    return 0;
}

void sjo_pool_free(sjo_pool *pool) {
    free(pool->body); free(pool->free_ids);
    pool->body = NULL; pool->free_ids = NULL; pool->n_free = 0;
}

uint32_t sjo_pool_alloc(sjo_pool *pool) { return pool->n_free ? pool->free_ids[--pool->n_free] : SJO_NO_BLOCK; }

void sjo_pool_release(sjo_pool *pool, uint32_t id) {
    if (id != SJO_NO_BLOCK && pool->n_free < pool->n_blocks) pool->free_ids[pool->n_free++] = id;
}

int sjo_seq_init(sjo_seq *s, const sjo_config *cfg, int n_layers, sjo_pool *pool) {
    int il, rc;
    uint32_t g;
    memset(s, 0, sizeof(*s));
    if (n_layers <= 0) return -100;
    s->cfg = *cfg;
    s->cfg.body = sjo_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (pool) {
        const sjo_config *pc = &pool->cfg;
        if (pool->n_layers != n_layers || pc->head_dim != cfg->head_dim || pc->n_head_kv != cfg->n_head_kv ||
            pc->group != cfg->group || pc->bits_k != cfg->bits_k || pc->bits_v != cfg->bits_v || pc->body != s->cfg.body)
            return -100;
    }
    s->n_layers = n_layers;
    s->pool = pool;
    s->layers = (sjo_layer *) calloc((size_t) n_layers, sizeof(sjo_layer));
    if (!s->layers) return -101;
    for (il = 0; il < n_layers; ++il) {
        rc = layer_setup(&s->layers[il], cfg, pool == NULL);
        if (rc) { s->n_layers = il; sjo_seq_free(s); return rc; }
    }
    if (pool) {
        s->blocks = (uint32_t *) malloc((size_t) s->layers[0].n_groups * sizeof(uint32_t));
        if (!s->blocks) { sjo_seq_free(s); return -101; }
        for (g = 0; g < s->layers[0].n_groups; ++g) s->blocks[g] = SJO_NO_BLOCK;
        for (il = 0; il < n_layers; ++il) {
            s->layers[il].body = pool->body + (size_t) il * pool->n_blocks * (size_t) cfg->n_head_kv * pool->lay.bytes;
            s->layers[il].blocks = s->blocks;
        }
    }
    sjo_policy_init(&s->pol, cfg->sink, cfg->tail, cfg->tail_max, (uint32_t) cfg->group, cfg->flush_chunk);
    s->n = 0;
    return 0;
}

static void seq_release(sjo_seq *s, uint32_t g0, uint32_t g1) {
    uint32_t g;
    if (!s->pool || !s->blocks) return;
    for (g = g0; g < g1 && g < s->layers[0].n_groups; ++g) {
        sjo_pool_release(s->pool, s->blocks[g]);
        s->blocks[g] = SJO_NO_BLOCK;
    }
}

static int seq_reserve(sjo_seq *s, uint32_t g0, uint32_t g1) {
    uint32_t g;
    if (!s->pool) return 0;
    if (g1 > s->layers[0].n_groups) return -109;
    for (g = g0; g < g1; ++g) {
        if (s->blocks[g] != SJO_NO_BLOCK) continue;
        s->blocks[g] = sjo_pool_alloc(s->pool);
        if (s->blocks[g] == SJO_NO_BLOCK) {
            while (g-- > g0) { sjo_pool_release(s->pool, s->blocks[g]); s->blocks[g] = SJO_NO_BLOCK; }
            return -110;
        }
    }
    return 0;
}

void sjo_seq_free(sjo_seq *s) {
    int il;
    if (s->layers) {
        if (s->pool && s->blocks) seq_release(s, 0, s->layers[0].n_groups);
        for (il = 0; il < s->n_layers; ++il) sjo_layer_free(&s->layers[il]);
    }
    free(s->layers); free(s->blocks);
    s->layers = NULL; s->blocks = NULL; s->n_layers = 0; s->n = 0;
}

void sjo_seq_reset(sjo_seq *s) {
    int il;
    for (il = 0; il < s->n_layers; ++il) sjo_layer_truncate(&s->layers[il], s->pol.B, s->cfg.sink, s->n, 0);
    seq_release(s, 0, s->layers[0].n_groups);
    sjo_policy_reset(&s->pol);
    s->n = 0;
}

static int seq_seal_commit(sjo_seq *s, const sjo_policy *before) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group;
    int il, rc;
    if (s->pol.B_pending > s->pol.B) {
        rc = seq_reserve(s, (s->pol.B - S) / G, (s->pol.B_pending - S) / G);
        if (rc) { s->pol = *before; return rc; }
        for (il = 0; il < s->n_layers; ++il) sjo_layer_seal(&s->layers[il], s->pol.B, s->pol.B_pending);
    }
    sjo_policy_commit(&s->pol);
    return 0;
}

int sjo_seq_begin_ubatch(sjo_seq *s, uint32_t pos0, uint32_t n_tokens) {
    const sjo_policy before = s->pol;
    if (pos0 > s->n) return -100;
    sjo_policy_begin_ubatch(&s->pol, pos0, n_tokens);
    return seq_seal_commit(s, &before);
}

void sjo_seq_store(sjo_seq *s, uint32_t pos, const float *k_rot, const float *v_rot) {
    const size_t stride = (size_t) s->cfg.n_head_kv * (size_t) s->cfg.head_dim;
    int il;
    for (il = 0; il < s->n_layers; ++il) sjo_layer_store(&s->layers[il], pos, k_rot + il * stride, v_rot + il * stride);
    if (pos + 1u > s->n) s->n = pos + 1u;
}

int sjo_seq_idle(sjo_seq *s, uint32_t keep_recent) {
    const sjo_policy before = s->pol;
    sjo_policy_idle(&s->pol, s->n, keep_recent);
    return seq_seal_commit(s, &before);
}

uint32_t sjo_seq_truncate(sjo_seq *s, uint32_t pos) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group, B_old = s->pol.B, n_old = s->n;
    uint32_t r;
    int il;
    r = sjo_policy_truncate(&s->pol, pos, NULL);
    if (r == SJO_NO_POS) return r;
    for (il = 0; il < s->n_layers; ++il) sjo_layer_truncate(&s->layers[il], B_old, s->pol.B, n_old, r);
    if (s->pol.B < B_old) seq_release(s, (s->pol.B - S) / G, (B_old - S) / G);
    if (r < s->n) s->n = r;
    return r;
}

void sjo_seq_attend_row(const sjo_seq *s, int il, const float *q_rot, int h, uint32_t qpos, float scale, float *out_rot) {
    sjo_layer_attend_row(&s->layers[il], s->pol.B, s->n, q_rot, h, qpos, scale, out_rot);
}

/* ------------------------------------------------------------------------------------------------ */
/* sequence state stream (sj_kvarn.h:1811-2034)                                                      */
/* ------------------------------------------------------------------------------------------------ */

uint64_t sjo_fnv1a(const void *p, size_t n, uint64_t h) {
    const uint8_t *b = (const uint8_t *) p;
    size_t i;
    for (i = 0; i < n; ++i) { h ^= b[i]; h *= UINT64_C(1099511628211); }
    return h;
}

static void le32(uint8_t *p, uint32_t v) { p[0] = (uint8_t) v; p[1] = (uint8_t) (v >> 8); p[2] = (uint8_t) (v >> 16); p[3] = (uint8_t) (v >> 24); }
static void le64(uint8_t *p, uint64_t v) { le32(p, (uint32_t) v); le32(p + 4, (uint32_t) (v >> 32)); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t) p[0] | (uint32_t) p[1] << 8 | (uint32_t) p[2] << 16 | (uint32_t) p[3] << 24; }
static uint64_t rd64(const uint8_t *p) { return (uint64_t) rd32(p) | (uint64_t) rd32(p + 4) << 32; }

static uint64_t codebook_id(int body, int bits_k, int bits_v) {
    uint64_t h = SJO_FNV0;
    if (body != SJO_BODY_TRELLIS) return 0;
    h = sjo_fnv1a(codebook(bits_k, 0), (size_t) (bits_k == 3 ? 512 : 256) * 2, h);
    h = sjo_fnv1a(codebook(bits_v, 1), (size_t) (bits_v == 3 ? 512 : 256) * 2, h);
    return h;
}

static size_t layer_payload(const sjo_config *c, const sjo_layout *lay, uint32_t n, uint32_t B) {
    const size_t H = (size_t) c->n_head_kv, rr = 2 * sjo_stage_row_bytes(c->staging, c->head_dim);
    const size_t sr = c->sink_type == SJO_SINK_F16 ? (size_t) c->head_dim * 4 : rr;
    const uint32_t ns = n < c->sink ? n : c->sink, nr = (B - c->sink) / (uint32_t) c->group, nt = n > B ? n - B : 0;
    return (size_t) ns * H * sr + (size_t) nr * H * lay->bytes + (size_t) nt * H * rr;
}

size_t sjo_seq_state_size(const sjo_seq *s) {
    return SJO_STATE_HDR + (size_t) s->n_layers * layer_payload(&s->cfg, &s->layers[0].lay, s->n, s->pol.B) + 8;
}

size_t sjo_state_size_max(const sjo_config *cfg, int n_layers) {
    sjo_config c = *cfg;
    sjo_layout lay;
    uint32_t B_all;
    size_t a, b;
    c.body = sjo_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (n_layers <= 0 || sjo_layout_init(&lay, c.head_dim, c.group, c.bits_k, c.bits_v, c.body)) return 0;
    B_all = c.n_ctx > c.sink ? c.sink + (uint32_t) c.group * ((c.n_ctx - c.sink + (uint32_t) c.group - 1u) / (uint32_t) c.group) : c.sink;
    a = layer_payload(&c, &lay, c.n_ctx, c.sink);
    b = layer_payload(&c, &lay, c.n_ctx, B_all);
    return SJO_STATE_HDR + (size_t) n_layers * (a > b ? a : b) + 8;
}

static const uint8_t state_magic[8] = { 'S', 'J', 'K', 'V', 'S', 'E', 'Q', 0 };

int sjo_seq_state_write(const sjo_seq *s, void *dst, size_t dst_size, size_t *written) {
    const sjo_config *c = &s->cfg;
    const size_t total = sjo_seq_state_size(s);
    const uint32_t S = c->sink, G = (uint32_t) c->group, B = s->pol.B, n = s->n;
    const int H = c->n_head_kv;
    uint8_t *o = (uint8_t *) dst, *w;
    uint32_t pos, g;
    int il, h;
    if (written) *written = 0;
    if (!s->layers || (!dst && dst_size)) return -100;
    if (s->pol.B_pending != s->pol.B) return -108;
    if (dst_size < total) return -102;
    memset(o, 0, SJO_STATE_HDR);
    memcpy(o, state_magic, 8);
    le32(o + 8, 1); le32(o + 12, 1); le32(o + 16, SJO_STATE_HDR);
    le32(o + 20, (uint32_t) c->head_dim); le32(o + 24, (uint32_t) c->n_head_kv); le32(o + 28, (uint32_t) c->group);
    le32(o + 32, c->sink); le32(o + 36, (uint32_t) c->sink_type); le32(o + 40, (uint32_t) c->bits_k);
    le32(o + 44, (uint32_t) c->bits_v); le32(o + 48, (uint32_t) c->body); le32(o + 52, (uint32_t) c->iters);
    le32(o + 56, (uint32_t) c->staging); le32(o + 60, c->tail); le32(o + 64, c->tail_max); le32(o + 68, c->flush_chunk);
    le32(o + 72, 1); le32(o + 76, (uint32_t) c->head_dim);
    le64(o + 80, codebook_id(c->body, c->bits_k, c->bits_v));
    le32(o + 88, (uint32_t) s->n_layers); le32(o + 92, n); le32(o + 96, B); le32(o + 100, s->pol.B_prev);
    le32(o + 104, (uint32_t) s->pol.draining);
    le64(o + 108, (uint64_t) (total - SJO_STATE_HDR - 8));
    w = o + SJO_STATE_HDR;
    for (il = 0; il < s->n_layers; ++il) {
        const sjo_layer *L = &s->layers[il];
        const size_t se = sink_entry_bytes(L), re = 2 * L->stage_bytes;
        for (pos = 0; pos < n && pos < S; ++pos)
            for (h = 0; h < H; ++h) { memcpy(w, sink_entry(L, pos, h), se); w += se; }
        for (g = 0; g < (B - S) / G; ++g)
            for (h = 0; h < H; ++h) { memcpy(w, sjo_layer_record(L, g, h), L->lay.bytes); w += L->lay.bytes; }
        for (pos = B; pos < n; ++pos)
            for (h = 0; h < H; ++h) { memcpy(w, ring_entry(L, pos, h), re); w += re; }
    }
    le64(w, sjo_fnv1a(o, (size_t) (w - o), SJO_FNV0));
    if (written) *written = total;
    return 0;
}

int sjo_state_peek(const void *src, size_t size, sjo_state_info *info) {
    const uint8_t *p = (const uint8_t *) src;
    sjo_state_info t;
    uint64_t payload;
    if (!src || !info) return -100;
    memset(&t, 0, sizeof(t));
    if (size < 8) return -103;
    if (memcmp(p, state_magic, 8)) return -104;
    if (size < 16) return -103;
    t.state_version = rd32(p + 8);
    t.format_version = rd32(p + 12);
    if (t.state_version != 1) return -105;
    if (size < SJO_STATE_HDR + 8) return -103;
    if (rd32(p + 16) != SJO_STATE_HDR) return -107;
    payload = rd64(p + 108);
    if (payload > (uint64_t) (size - SJO_STATE_HDR - 8)) return -103;
    t.total_bytes = SJO_STATE_HDR + (size_t) payload + 8;
    if (sjo_fnv1a(p, t.total_bytes - 8, SJO_FNV0) != rd64(p + t.total_bytes - 8)) return -107;
    if (t.format_version != 1) return -106;
    t.cfg.head_dim = (int) rd32(p + 20); t.cfg.n_head_kv = (int) rd32(p + 24); t.cfg.group = (int) rd32(p + 28);
    t.cfg.sink = rd32(p + 32); t.cfg.sink_type = (int) rd32(p + 36); t.cfg.bits_k = (int) rd32(p + 40);
    t.cfg.bits_v = (int) rd32(p + 44); t.cfg.body = (int) rd32(p + 48); t.cfg.iters = (int) rd32(p + 52);
    t.cfg.staging = (int) rd32(p + 56); t.cfg.tail = rd32(p + 60); t.cfg.tail_max = rd32(p + 64);
    t.cfg.flush_chunk = rd32(p + 68); t.rotation = rd32(p + 72); t.rotation_n = rd32(p + 76);
    t.codebook_id = rd64(p + 80); t.n_layers = (int) rd32(p + 88); t.n = rd32(p + 92); t.B = rd32(p + 96);
    t.B_prev = rd32(p + 100); t.draining = rd32(p + 104);
    *info = t;
    return 0;
}

int sjo_seq_state_read(sjo_seq *s, const void *src, size_t size) {
    const sjo_config *c = &s->cfg;
    const uint8_t *r;
    sjo_state_info t;
    uint32_t S, G, n_rec, pos, g, held = 0;
    int il, h, rc;
    if (!s->layers) return -100;
    rc = sjo_state_peek(src, size, &t);
    if (rc) return rc;
    if (t.cfg.head_dim != c->head_dim) return -120;
    if (t.cfg.n_head_kv != c->n_head_kv) return -121;
    if (t.cfg.group != c->group) return -122;
    if (t.cfg.sink != c->sink || t.cfg.sink_type != c->sink_type) return -123;
    if (t.cfg.bits_k != c->bits_k || t.cfg.bits_v != c->bits_v) return -124;
    if (t.cfg.body != c->body) return -125;
    if (t.cfg.iters != c->iters) return -126;
    if (t.cfg.staging != c->staging) return -127;
    if (t.cfg.tail != c->tail || t.cfg.tail_max != c->tail_max || t.cfg.flush_chunk != c->flush_chunk) return -128;
    if (t.rotation != 1 || t.rotation_n != (uint32_t) c->head_dim) return -129;
    if (t.codebook_id != codebook_id(c->body, c->bits_k, c->bits_v)) return -130;
    if (t.n_layers != s->n_layers) return -131;
    S = c->sink; G = (uint32_t) c->group;
    if (t.B < S || (t.B - S) % G || t.B_prev < S || t.B_prev > t.B || (t.B_prev - S) % G || t.draining > 1 ||
        (t.B > S && t.B > t.n)) return -107;
    if (t.total_bytes != SJO_STATE_HDR + (size_t) s->n_layers * layer_payload(c, &s->layers[0].lay, t.n, t.B) + 8) return -107;
    n_rec = (t.B - S) / G;
    if (t.n > c->n_ctx || n_rec > s->layers[0].n_groups || (t.n > t.B && t.n - t.B > s->layers[0].cap)) return -109;
    if (s->pool) {
        for (g = 0; g < s->layers[0].n_groups; ++g) held += s->blocks[g] != SJO_NO_BLOCK;
        if (s->pool->n_free + held < n_rec) return -110;
    }
    sjo_seq_reset(s);
    if (seq_reserve(s, 0, n_rec)) return -110;
    r = (const uint8_t *) src + SJO_STATE_HDR;
    for (il = 0; il < s->n_layers; ++il) {
        sjo_layer *L = &s->layers[il];
        const size_t se = sink_entry_bytes(L), re = 2 * L->stage_bytes;
        for (pos = 0; pos < t.n && pos < S; ++pos)
            for (h = 0; h < c->n_head_kv; ++h) { memcpy(sink_entry(L, pos, h), r, se); r += se; }
        for (g = 0; g < n_rec; ++g)
            for (h = 0; h < c->n_head_kv; ++h) { memcpy(sjo_layer_record(L, g, h), r, L->lay.bytes); r += L->lay.bytes; }
        for (pos = t.B; pos < t.n; ++pos)
            for (h = 0; h < c->n_head_kv; ++h) { memcpy(ring_entry(L, pos, h), r, re); r += re; }
    }
    s->pol.B = s->pol.B_pending = t.B;
    s->pol.B_prev = t.B_prev;
    s->pol.draining = (int) t.draining;
    s->n = t.n;
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* test-support generators                                                                           */
/* ------------------------------------------------------------------------------------------------ */

/* xorshift64 (13, 7, 17), top bits (tests/vector_inputs.h:8-11) */
static uint32_t xs_next(uint64_t *s) {
    *s ^= *s << 13; *s ^= *s >> 7; *s ^= *s << 17;
    return (uint32_t) (*s >> 11);
}
/* sum of four 10-bit uniforms, centred (tests/vector_inputs.h:14-18) */
static int32_t xs_gauss(uint64_t *s) {
    int32_t a = 0;
    int i;
    for (i = 0; i < 4; ++i) a += (int32_t) (xs_next(s) & 1023u) - 512;
    return a;
}
static float xs_value(uint64_t *s, int chf, int tf) { return (float) (xs_gauss(s) * chf * tf) * (1.0f / 4096.0f); }

void sjo_vec_fill_group(int D, int G, uint32_t seed, uint16_t *K, uint16_t *V) {
    /* tests/vector_inputs.h:27-39 */
    uint64_t s = UINT64_C(0x9E3779B97F4A7C15) ^ seed;
    int side, t, d;
    int *chf = (int *) malloc((size_t) D * sizeof(int));
    for (side = 0; side < 2; ++side) {
        uint16_t *X = side ? V : K;
        for (d = 0; d < D; ++d) {
            const int outlier = (xs_next(&s) % 100u) < 3u;
            chf[d] = outlier ? 24 + (int) (xs_next(&s) & 7u) : 1 + (int) (xs_next(&s) & 3u);
        }
        for (t = 0; t < G; ++t) {
            const int tf = 1 + (int) (xs_next(&s) & 3u);
            for (d = 0; d < D; ++d) X[(size_t) t * D + d] = sjo_f32_to_f16(xs_value(&s, chf[d], tf));
        }
    }
    free(chf);
}

void sjo_vec_fill_rows(int rows, int n, float *x) {
    /* tests/vector_inputs.h:42-50 */
    uint64_t s = UINT64_C(0xD1B54A32D192ED03);
    int r, i;
    for (r = 0; r < rows; ++r) {
        const int tf = 1 + (int) (xs_next(&s) & 7u);
        for (i = 0; i < n; ++i) x[(size_t) r * n + i] = xs_value(&s, 1, tf);
        if (r == rows - 1)
            for (i = 0; i < n; ++i) x[(size_t) r * n + i] = 0.0f;
    }
}

/* splitmix64 finaliser (tests/test_state.c:33-38) */
static uint64_t sm_mix(uint64_t x) {
    x += UINT64_C(0x9E3779B97F4A7C15);
    x = (x ^ (x >> 30)) * UINT64_C(0xBF58476D1CE4E5B9);
    x = (x ^ (x >> 27)) * UINT64_C(0x94D049BB133111EB);
    return x ^ (x >> 31);
}

float sjo_st_val(uint32_t seed, uint32_t variant, uint32_t pos, uint32_t i, int side) {
    /* tests/test_state.c:40-45 */
    const uint64_t h = sm_mix(((uint64_t) seed << 40) ^ ((uint64_t) variant << 36) ^ ((uint64_t) pos << 16) ^
                              ((uint64_t) i << 1) ^ (uint64_t) side);
    const int32_t g = (int32_t) (h & 1023u) + (int32_t) ((h >> 10) & 1023u) - 1024;
    const int sc = (i % 41u) == 0 ? 24 : 1 + (int) ((h >> 20) & 3u);
    return (float) (g * sc) * (1.0f / 4096.0f);
}

int sjo_st_grow(sjo_seq *q, uint32_t seed, uint32_t edit_from, uint32_t edit_variant, uint32_t from, uint32_t to,
                uint32_t pattern) {
    /* tests/test_state.c:55-74: ubatches of a deterministic size pattern */
    const size_t row = (size_t) q->n_layers * (size_t) q->cfg.n_head_kv * (size_t) q->cfg.head_dim;
    float *k = (float *) malloc(row * sizeof(float)), *v = (float *) malloc(row * sizeof(float));
    uint32_t pos = from, step = 0;
    int rc = 0;
    while (pos < to) {
        uint32_t n = pattern == 0 ? 1u : (step % 5u == 4u ? 1u + (pattern * 7u + step * 13u) % 64u : 1u + (step + pattern) % 4u);
        uint32_t i;
        size_t j;
        if (pos + n > to) n = to - pos;
        rc = sjo_seq_begin_ubatch(q, pos, n);
        if (rc) break;
        for (i = 0; i < n; ++i) {
            const uint32_t p = pos + i, var = p >= edit_from ? edit_variant : 0u;
            for (j = 0; j < row; ++j) { k[j] = sjo_st_val(seed, var, p, (uint32_t) j, 0); v[j] = sjo_st_val(seed, var, p, (uint32_t) j, 1); }
            sjo_seq_store(q, p, k, v);
        }
        pos += n;
        step++;
    }
    free(k); free(v);
    return rc;
}
