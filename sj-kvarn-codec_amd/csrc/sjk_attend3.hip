// sjk_attend3.hip - streaming decode attention on the matrix cores (4/4 scalar and 3/3, 3/2, 2/2
// trellis bodies, D = 256).
//
// One launch covers the whole context of every KV head; a second, small launch merges the partials.
// The query rows of one KV head (decode width x GQA group <= 16) are the 16 rows of every MFMA tile,
// so each record and each staging row is read from HBM once per call. Reference decode:
// sj_kvarn.h:1178-1207; attention loop: sj_kvarn.h:1535-1564.
//
// Both kernels have record workgroups and row workgroups (the fp16 sink and the staging tail); every
// workgroup ends with one (m, l, O[16][256]) partial (m in log2 units).
//
// Codes as MFMA operands. The 4-bit codes enter v_mfma_f32_16x16x32_f16 as fp16 subnormals: masking a
// fragment word with 0x000F000F yields the fp16 pair (c0 * 2^-24, c4 * 2^-24), with 0x00F000F0
// (c1 * 2^-20, c5 * 2^-20); the other four nibbles after an 8-bit shift. The power of two is removed after
// the product. With
//   K[t,d] = (c*Kscale[d] + Kzero[d]) * Ktok[t]  ->  S[q,t] = Ktok[t] * (sum_d Q'[q,d]*c + sum_d Q[q,d]*Kzero[d]),
//   V[t,d] = (c*Vscale[t] + Vzero[t]) * Vch[d]   ->  O[q,d] += Vch[d] * (sum_t P'[q,t]*c + sum_t P[q,t]*Vzero[t]),
// Q' = Q*Kscale is split into fp16 hi + lo parts (two MFMAs; ~22 significant bits, within fp32-accumulation
// error of the reference's fp32 sums, sj_kvarn.h:1288-1311); P' = P*Vscale is rounded to fp16 once (an
// unbiased 2^-12 relative error per weight, which averages out over the tokens of an output), and the
// zero-point sums enter in fp32.
//
// 4/4 bodies (attend4_kernel, a4_records): one workgroup of 8 wavefronts per CU; every record wavefront
// streams its own records through a ring of LDS chunks filled by global_load_lds (see the section on
// streaming record wavefronts).
//
// Trellis bodies (attend3_kernel, a3_trellis; channel-major Viterbi streams, sj_kvarn.h:870-900): the
// value of (token t, channel d) is codebook[window], window = the code of t over the 6 stream bits before
// it. The codebook entries are exact fp16 MFMA operands, so the same Q' / P' folding applies. One LDS
// lookup in a "pair table" decodes two tokens t, t+1 of one channel: its index is the 6 + 2 * bits stream
// bits that end with the code of t+1, its entry the fp16 values of both windows. For V the looked-up word
// is already the B operand (k = tokens); for K (k = channels) two words are interleaved by v_perm. The
// four wavefronts of a workgroup share one record in LDS (the next one is already in registers); QK and
// the softmax are split by tokens (a wavefront owns 32 tokens: K tile tt, row r is token 32w + 2r + tt, so
// that its accumulator entries are 8 consecutive tokens per lane, in PV slot order), the PV product by
// channels.
//
// Row workgroups: independent wavefronts, each taking 16-position chunks of the sink or the tail (fp16
// rows, or tq6_0 rows dequantized as centroid x block norm, sj_kvarn.h:1249-1260). tq6_0 K|V rows are
// staged in the wavefront's LDS slice and decoded two channels per lookup in a centroid pair table (fp16
// hi / lo of both codes); fp16 rows are read from HBM where they are used. K values go through
// v_mfma_f32_16x16x32_f16 (Q hi + lo, K hi + lo for tq6_0), V values through v_mfma_f32_16x16x16_f16,
// the tq6_0 block norms are applied to the K accumulator and folded into P for V.
#include "sjk_dev.h"

#include <atomic>
#include <type_traits>

namespace sjk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int A3_NT = 256;
constexpr int A3_Q = 16;
constexpr int A3_D = 256;
constexpr int A3_CH = 16;                        // positions per row chunk
constexpr int A3_STAGE = A3_CH * 2 * 2 * SJKVARN_TQ6_BLOCK_BYTES;   // LDS bytes per wavefront: 16 tq6_0 K | V rows
constexpr int A3_PSTRIDE = A3_Q * (A3_D + 2);    // floats per partial

// record layout at head dimension D (256 unless given), G = 128 with BK / BV bits per K / V code
// (sj_kvarn.h:771-790): K payload | V payload | Kscale[D] | Kzero[D] | Ktok[G] | Vch[D] | Vscale[G] | Vzero[G]
template <int BK, int BV, int D = A3_D> struct RecLay {
    static constexpr int VPAY = 16 * D * BK, KSC = VPAY + 16 * D * BV, KZE = KSC + 2 * D, KTOK = KZE + 2 * D,
                         VCH = KTOK + 256, VSC = VCH + 2 * D, VZE = VSC + 256, BYTES = VZE + 256;
};
constexpr int R_VPAY = RecLay<4, 4>::VPAY, R_KSC = RecLay<4, 4>::KSC, R_KZE = RecLay<4, 4>::KZE,
              R_KTOK = RecLay<4, 4>::KTOK, R_VCH = RecLay<4, 4>::VCH, R_VSC = RecLay<4, 4>::VSC,
              R_VZE = RecLay<4, 4>::VZE, R_BYTES = RecLay<4, 4>::BYTES;
static_assert(R_BYTES == 35072 && RecLay<3, 3>::BYTES == 26880 && RecLay<3, 2>::BYTES == 22784 &&
              RecLay<2, 2>::BYTES == 18688, "record sizes of sj_kvarn.h:792-794");

// 4/4 record layout at head dimension D (128 or 256), G = 128 (sj_kvarn.h:771-790)
template <int D> struct RecLay4 {
    static constexpr int VPAY = 64 * D, KSC = 128 * D, KZE = KSC + 2 * D, KTOK = KZE + 2 * D, VCH = KTOK + 256,
                         VSC = VCH + 2 * D, VZE = VSC + 256, BYTES = VZE + 256;
};
static_assert(RecLay4<256>::BYTES == R_BYTES && RecLay4<256>::VCH == R_VCH && RecLay4<128>::BYTES == 17920,
              "4/4 record sizes of sj_kvarn.h:792-794 (D = 256, 128)");

// Trellis pair tables: entry e (6 + 2B bits of a channel stream, oldest bit first) holds the fp16
// codebook values of the two windows it contains, cb[e & (2^(6+B) - 1)] | cb[e >> B] << 16.
template <int B> struct PairTab { uint32_t v[1 << (6 + 2 * B)]; };
template <int B, int NC>
constexpr PairTab<B> make_pairs(const uint16_t (&cb)[NC]) {
    PairTab<B> t{};
    for (uint32_t e = 0; e < (1u << (6 + 2 * B)); ++e)
        t.v[e] = (uint32_t) cb[e & ((1u << (6 + B)) - 1u)] | ((uint32_t) cb[e >> B] << 16);
    return t;
}
constexpr uint16_t k_cb3k[512] = SJK_CB3_K_INIT, k_cb3v[512] = SJK_CB3_V_INIT;
constexpr uint16_t k_cb2k[256] = SJK_CB2_K_INIT, k_cb2v[256] = SJK_CB2_V_INIT;
static __device__ const PairTab<3> g_pair3k = make_pairs<3>(k_cb3k);
static __device__ const PairTab<3> g_pair3v = make_pairs<3>(k_cb3v);
static __device__ const PairTab<2> g_pair2k = make_pairs<2>(k_cb2k);
static __device__ const PairTab<2> g_pair2v = make_pairs<2>(k_cb2v);
template <int B, bool IS_V> SJK_DEV const uint32_t * pair_tab() {
    if (B == 3) return IS_V ? g_pair3v.v : g_pair3k.v;
    return IS_V ? g_pair2v.v : g_pair2k.v;
}

struct A3Args {
    sjk_hip_view v;
    uint32_t N, qpos0;
    // query rows of a KV head: row r = iq * gq + j is query position qpos0 + iq, query head h * gq + j; this job
    // (a tile) takes rows row0 .. row0 + n_rows - 1 (n_rows <= 16, the rows of an MFMA tile)
    int n_q, n_head, gq, n_rows, row0;
    float sc2;                    // scale * log2(e): scores in log2 units
    const float * q;
    float * out;
    float * part;                 // [H][n_wg][A3_Q][A3_D + 2]
    uint32_t sink_end, body_end, pend;
    int n_rec;                    // sealed records per KV head in [S, body_end)
    int n_chunk, sink_chunks;     // row chunks per KV head: sink chunks first, then the tail
    int n_row_wg, n_rec_wg, n_wg; // workgroups per KV head
    int rec_per_wg;
    int slots, rec_slots;         // 4/4 kernel: CU slots per KV head (one workgroup each), of them record slots
    int rec_a, rec_b;             // 4/4 kernel: records per wavefront (rec_b unused)
};

// Q' operands are read in the QK phase, P' operands in the PV phase of a record, with a barrier between
// the last QK read and the first P' write, so they share their LDS
union QPOps {
    uint16_t qb[2][8][4][A3_Q][8];               // Q' hi / lo in B-operand order [hl][k-step][lane group][query][slot]
    u4 pa[4][64];                                // P' A operands (fp16) of the four 32-token k-steps
};


template <int NW> struct RowLdsT {
    alignas(16) uint8_t stage[NW][A3_STAGE];     // per wavefront: 16 staged tq6_0 rows (K | V)
    alignas(16) uint16_t qb[2][8][4][A3_Q][8];   // Q hi / lo in B-operand order
    u2 pt[4096];                                 // tq6_0 pair table (tq6_pairs8)
    float cent[64];                              // tq6_0 centroids, staged once for the table build
};

// A trellis record as it sits in LDS: each channel's stream (16 x bits bytes) padded by one dword, so that the
// stream words one instruction reads for lanes of different channel groups fall in different banks (at the
// record's own 12- or 8-dword stride the four lane groups of a K read share their banks), then the scale tables,
// 16-byte aligned and in the record's order (sj_kvarn.h:771-790).
template <int BK, int BV, int D = A3_D> struct TrPad {
    static constexpr int KSTR = 16 * BK + 4, VSTR = 16 * BV + 4;
    static constexpr int VPAY = D * KSTR, KSC = VPAY + D * VSTR, KZE = KSC + 2 * D, KTOK = KZE + 2 * D, VCH = KTOK + 256,
                         VSC = VCH + 2 * D, VZE = VSC + 256, BYTES = VZE + 256;
    static_assert(KSC % 16 == 0 && KZE - KSC == RecLay<BK, BV, D>::KZE - RecLay<BK, BV, D>::KSC &&
                  BYTES - KSC == RecLay<BK, BV, D>::BYTES - RecLay<BK, BV, D>::KSC, "scale tables of the record, 16-byte aligned");
};

template <int BK, int BV, int D = A3_D> struct TrLds {
    uint32_t zero[4];                            // read (and masked) before channel 0's stream
    alignas(16) uint8_t rec[TrPad<BK, BV, D>::BYTES];
    alignas(16) uint32_t tk[1 << (6 + 2 * BK)];  // K / V pair tables
    alignas(16) uint32_t tv[1 << (6 + 2 * BV)];
    alignas(16) QPOps op;
    float corr[4][A3_Q];
    float wmax[4][A3_Q];
    float cvp[4][A3_Q];
};

template <typename RL, int NW = 4> struct A3LdsT {
    union {
        RL r;
        RowLdsT<NW> w;
    };
    alignas(16) float wm[NW][A3_Q];              // per-wave softmax state at the merge
    alignas(16) float wl[NW][A3_Q];
    alignas(16) float wf[NW][A3_Q];              // merge factors exp2(m_w - M) per wave and query
};

SJK_DEV f4 mfma32(const u4 & a, const u4 & b, const f4 & c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

SJK_DEV f4 mfma16(const u2 & a, const u2 & b, const f4 & c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
}

SJK_DEV float h2f(uint32_t bits16) { return (float) __builtin_bit_cast(_Float16, (uint16_t) bits16); }

// (x0, x1) as fp16 pairs {hi, lo}: hi = RN16(x), lo = RN16(x - hi)
SJK_DEV u2 split2(float x0, float x1) {
    const _Float16 a = (_Float16) x0, b = (_Float16) x1;
    const _Float16 c = (_Float16) (x0 - (float) a), d = (_Float16) (x1 - (float) b);
    return u2{(uint32_t) __builtin_bit_cast(uint16_t, a) | ((uint32_t) __builtin_bit_cast(uint16_t, b) << 16),
              (uint32_t) __builtin_bit_cast(uint16_t, c) | ((uint32_t) __builtin_bit_cast(uint16_t, d) << 16)};
}

// v_fma_mix: fp32 a times the low / high fp16 half of h2 (plus fp32 c), the exact product rounded once, to
// fp32. Inline asm: never pass these a register written by an MFMA (no hazard wait states are inserted for
// asm operands).
SJK_DEV float mul_lo(float a, uint32_t h2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(h2));
    return r;
}
SJK_DEV float mul_hi(float a, uint32_t h2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(h2));
    return r;
}
SJK_DEV float fma_lo(float a, uint32_t h2, float c) { return __builtin_fmaf(a, h2f(h2 & 0xFFFFu), c); }
SJK_DEV float fma_hi(float a, uint32_t h2, float c) { return __builtin_fmaf(a, h2f(h2 >> 16), c); }

// fp16 pair {RN16(a0 * s.lo), RN16(a1 * s.hi)}: v_fma_mixlo / mixhi round the exact product once and write
// one half of the destination, keeping the other (the mixlo result's high half is whatever the register
// held, until the mixhi writes it). The compiler inserts no hazard wait states around inline asm (it does not
// see a VALU instruction there), so the asm gives them itself:
// * the pairs are MFMA operands, read by the next MFMA as soon as they are written, and a VALU write needs two
//   wait states before an MFMA reads the register: s_nop 1 ends the asm. Without it the 4/4 kernel's products
//   read stale operand halves whenever the scheduler placed an MFMA one instruction after a pair's last write
//   (wrong, run-to-run varying attention output);
// * a0 and a1 are often exp2 results just computed, and a transcendental result needs one wait state before
//   another VALU instruction reads it: s_nop 0 begins each instruction's asm.
SJK_DEV uint32_t mul_pk(float a0, float a1, uint32_t s) {
    uint32_t d;
    asm("s_nop 0\n\tv_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(d) : "v"(a0), "v"(s));
    asm("s_nop 0\n\tv_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\ts_nop 1" : "+v"(d) : "v"(a1), "v"(s));
    return d;
}

// (a0 * s.lo, a1 * s.hi) as fp16 pairs {hi, lo}: hi = RN16(x), lo = RN16(x - hi) with the exact x (hi + lo
// within 2^-22 of each product, less where lo is subnormal); MFMA operands as mul_pk's
SJK_DEV u2 mul_split(float a0, float a1, uint32_t s) {
    const uint32_t hi = mul_pk(a0, a1, s);
    uint32_t lo;
    asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,1,1]" : "=v"(lo) : "v"(a0), "v"(s), "v"(hi));
    asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,1,1] op_sel_hi:[0,1,1]\n\ts_nop 1" : "+v"(lo) : "v"(a1), "v"(s), "v"(hi));
    return u2{hi, lo};
}

// Row exchange between two registers: v_permlane16_swap_b32 swaps the odd 16-lane rows of x with the even
// rows of y, v_permlane32_swap_b32 the upper 32 lanes of x with the lower 32 of y (no LDS round trip, unlike
// a lane shuffle). Written out as asm because this toolchain's builtin returns the first register for both
// results; s_nop 1 gives the wait states a VALU write needs before the swap reads it. Never pass an MFMA result.
SJK_DEV void swap16(uint32_t & x, uint32_t & y) { asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y)); }
SJK_DEV void swap32(uint32_t & x, uint32_t & y) { asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y)); }

// sum / max over the four 16-lane rows of a wavefront (the MFMA lane groups g), (r0 + r1) + (r2 + r3), the
// same value in every lane
SJK_DEV float rows_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap16(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b)), d = c;
    swap32(c, d);
    return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}
SJK_DEV float rows_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap16(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b))), d = c;
    swap32(c, d);
    return fmaxf(__builtin_bit_cast(float, c), __builtin_bit_cast(float, d));
}

// max / sum over all 64 lanes: DPP rotations inside the rows, then across the rows (same value in every lane)
SJK_DEV float wave_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xF, 0xF, false)));
    return rows_max(v);
}
SJK_DEV float wave_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xF, 0xF, false));
    return rows_sum(v);
}

// unsigned max over all 64 lanes: DPP rotations inside the rows, then across the rows
SJK_DEV uint32_t wave_umax(uint32_t v) {
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x128, 0xF, 0xF, false));    // row_ror:8
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x124, 0xF, 0xF, false));    // row_ror:4
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x122, 0xF, 0xF, false));    // row_ror:2
    v = max(v, (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x121, 0xF, 0xF, false));    // row_ror:1
    uint32_t a = v, b = v;
    swap16(a, b);
    uint32_t c = max(a, b), d = c;
    swap32(c, d);
    return max(c, d);
}

// Power of two 2^k for the P' operands of one record: with vmax = max_t Vscale[t] in [2^(e-1), 2^e),
// P' = P * Vscale * 2^k (P <= 1, k = 14 - e) stays below 2^14 and the small weights stay clear of the
// fp16 subnormal range, where they would lose their low bits. Returns 2^k (uniform over
// the wave) and inv = 2^-k, by which the product is scaled back. vsc: the record's Vscale[128] in LDS.
SJK_DEV float pv_scale(const uint8_t * vsc, int lane, float & inv) {
    const uint32_t wv = *(const uint32_t *) (vsc + 4 * lane);       // Vscale of tokens 2 lane, 2 lane + 1 (>= 0)
    const uint32_t mx = wave_umax(max(wv & 0xFFFFu, wv >> 16));       // non-negative halves order like their bits
    const int e = __builtin_amdgcn_frexp_expf(h2f(mx));
    inv = __builtin_amdgcn_ldexpf(1.0f, e - 14);
    return __builtin_amdgcn_ldexpf(1.0f, 14 - e);
}

// Issue priority from a wavefront's progress through its own work (first quarter 3, ..., last quarter 0).
// Wavefronts that share a SIMD are not issued evenly at equal priority: one finishes well before the other,
// which then runs alone at a lower rate (the loop ends of the 8 record wavefronts of a CU spread by ~6 us).
// Ranking by progress lets the one behind catch up, so that they end together.
SJK_DEV void prio_by_progress(int done, int total) {
    const int q = (4 * done) / (total > 0 ? total : 1);
    if (q <= 0) __builtin_amdgcn_s_setprio(3);
    else if (q == 1) __builtin_amdgcn_s_setprio(2);
    else if (q == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

SJK_DEV void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// query row n of the tile for KV head h: (position index, global head); rows past n_rows are dead (masked)
template <int D = A3_D> SJK_DEV const float * q_row(const A3Args & a, int h, int n) {
    const int r = a.row0 + (n < a.n_rows ? n : 0);
    const int iq = r / a.gq, hq = h * a.gq + r % a.gq;
    return a.q + ((size_t) iq * a.n_head + hq) * D;
}

// causal end of query row n of the tile (positions < qend are visible; 0 for a dead row); non-decreasing in n
// over the live rows
SJK_DEV uint32_t q_end(const A3Args & a, int n) {
    if (n >= a.n_rows) return 0u;
    const uint32_t qpos = a.qpos0 + (uint32_t) ((a.row0 + n) / a.gq);
    return qpos + 1 < a.N ? qpos + 1 : a.N;
}

// online softmax over K values per lane (log2 units); returns alpha for the old state
template <int K>
SJK_DEV float softmax_update(float * sc, float & m_run, float & l_run) {
    float mloc = sc[0];
#pragma unroll
    for (int k = 1; k < K; ++k) mloc = fmaxf(mloc, sc[k]);
    mloc = rows_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const bool any = m_new != -__builtin_inff();
    const float alpha = any ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        sc[k] = any ? __builtin_amdgcn_exp2f(sc[k] - m_new) : 0.0f;
        psum += sc[k];
    }
    psum = rows_sum(psum);
    m_run = m_new;
    l_run = l_run * alpha + psum;
    return alpha;
}

// merge the four wavefronts' (m, l, O) into the workgroup partial. Lane (n, g) of wave w holds
// O[j][i] = (query 4g + i, channel chan(j, n)) scaled by oscale (D / 16 tiles j).
template <int D, typename Lds, typename Chan>
SJK_DEV void write_partial(const A3Args & a, Lds & s, float * ob, int h, int wgi, const f4 * O, float m_run,
                           float l_run, float oscale, Chan chan) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    __syncthreads();
    if (g == 0) { s.wm[w][n] = m_run; s.wl[w][n] = l_run; }
    __syncthreads();
    float fac[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * g + i;
        const float M = fmaxf(fmaxf(s.wm[0][q], s.wm[1][q]), fmaxf(s.wm[2][q], s.wm[3][q]));
        fac[i] = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(s.wm[w][q] - M) * oscale;
    }
    for (int k = 0; k < 4; ++k) {
        if (w == k) {
#pragma unroll
            for (int j = 0; j < D / 16; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float & dst = ob[(4 * g + i) * D + chan(j, n)];
                    dst = (k == 0 ? 0.0f : dst) + O[j][i] * fac[i];
                }
        }
        __syncthreads();
    }
    float * part = a.part + ((size_t) h * a.n_wg + wgi) * (A3_Q * (D + 2));
    for (int e = tid; e < A3_Q * D; e += A3_NT) part[(e / D) * (D + 2) + 2 + (e % D)] = ob[e];
    if (tid < A3_Q) {
        const float M = fmaxf(fmaxf(s.wm[0][tid], s.wm[1][tid]), fmaxf(s.wm[2][tid], s.wm[3][tid]));
        float Ls = 0.0f;
        if (M != -__builtin_inff())
            for (int k = 0; k < 4; ++k) Ls += s.wl[k][tid] * __builtin_amdgcn_exp2f(s.wm[k][tid] - M);
        part[tid * (D + 2)] = M;
        part[tid * (D + 2) + 1] = Ls;
    }
}

// The merge of workgroups with 16 KB of LDS per wavefront for its O tiles, in two steps.
// partial_put: the wavefront's O tiles, unscaled, in their register order ([tile j][lane] x 4 floats, bank-
// conflict free) at its area bw, and its (m, l). The area must be free: a record wavefront's own stream
// buffers once its stream is done (so that it writes while the others still run), else after a barrier.
// (NJ O tiles: D / 16)
template <int NJ, typename Lds>
SJK_DEV void partial_put(Lds & s, f4 * bw, const f4 * O, float m_run, float l_run) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < NJ; ++j) bw[j * 64 + lane] = O[j];
    if (g == 0) { s.wm[w][n] = m_run; s.wl[w][n] = l_run; }
}

// partial_gather (every wavefront, after its partial_put): the factors exp2(m_w - M) of every wave and
// query, then thread t sums channel d = t % D of queries QT(t / D) .. +QT-1 (QT = 16 D / (64 NW): 8 at
// D = 256 and NW = 8) over the waves' areas (wave w2's area at buf + w2 * stride f4s; inv(d, j, n): the tile j
// and column n that hold channel d) and writes it to the partial, with the partial's (M, L).
template <int D, typename Lds, typename Inv>
SJK_DEV void partial_gather(const A3Args & a, Lds & s, const f4 * buf, int stride, int h, int wgi, Inv inv) {
    constexpr int NW = sizeof(s.wm) / sizeof(s.wm[0]);
    constexpr int QT = A3_Q * D / (64 * NW);     // queries per thread
    static_assert(QT % 4 == 0 && A3_Q % QT == 0, "whole 4-query groups per thread");
    const int tid = threadIdx.x;
    float * part = a.part + ((size_t) h * a.n_wg + wgi) * (A3_Q * (D + 2));
    __syncthreads();
    if (tid < NW * A3_Q) {
        const int w2 = tid / A3_Q, q = tid % A3_Q;
        float M = s.wm[0][q];
#pragma unroll
        for (int k = 1; k < NW; ++k) M = fmaxf(M, s.wm[k][q]);
        const float f = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(s.wm[w2][q] - M);
        s.wf[w2][q] = f;
        if (w2 == 0) {
            float Ls = 0.0f;
            if (M != -__builtin_inff())
                for (int k = 0; k < NW; ++k) Ls += s.wl[k][q] * __builtin_amdgcn_exp2f(s.wm[k][q] - M);
            part[q * (D + 2)] = M;
            part[q * (D + 2) + 1] = Ls;
        }
    }
    __syncthreads();
    const int d = tid % D, q0 = QT * (tid / D);
    int j, nn;
    inv(d, j, nn);
    f4 acc[QT / 4];
#pragma unroll
    for (int k = 0; k < QT / 4; ++k) acc[k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2)
#pragma unroll
        for (int k = 0; k < QT / 4; ++k) {
            const int gg = q0 / 4 + k;
            const f4 f = *(const f4 *) &s.wf[w2][4 * gg];
            acc[k] = acc[k] + buf[w2 * stride + j * 64 + 16 * gg + nn] * f;
        }
#pragma unroll
    for (int q = 0; q < QT; ++q) part[(q0 + q) * (D + 2) + 2 + d] = acc[q >> 2][q & 3];
}

// ------------------------------------------------------------------------------------------------
// record workgroups
// ------------------------------------------------------------------------------------------------

// partial of a (trellis) record workgroup whose waves share m and hold disjoint channel slices of O: lane (n, g) of wave w
// holds O[4g + i] of channel 16(NJW w + jj) + n (NJW = D / 64 tiles a wave; scaled by osc); l is the sum of the waves' parts
template <int D, typename Lds>
SJK_DEV void write_partial_cs(const A3Args & a, Lds & S, int h, int wgi, const f4 * O, float m_run, float l_run,
                              float osc) {
    constexpr int NJW = D / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    __syncthreads();
    if (g == 0) S.wl[w][n] = l_run;
    __syncthreads();
    float * part = a.part + ((size_t) h * a.n_wg + wgi) * (A3_Q * (D + 2));
#pragma unroll
    for (int jj = 0; jj < NJW; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[(4 * g + i) * (D + 2) + 2 + 16 * (NJW * w + jj) + n] = O[jj][i] * osc;
    if (tid < A3_Q) {
        part[tid * (D + 2)] = m_run;
        part[tid * (D + 2) + 1] = (S.wl[0][tid] + S.wl[1][tid]) + (S.wl[2][tid] + S.wl[3][tid]);
    }
}

// ------------------------------------------------------------------------------------------------
// streaming record wavefronts (4/4 scalar body)
// ------------------------------------------------------------------------------------------------
//
// Every wavefront of a record workgroup (8 wavefronts, one workgroup per CU, two wavefronts per SIMD) owns
// a contiguous range of records of one KV head and streams them through its own ring of A4_SLOTS 4 KB
// chunks in LDS; there are no barriers between the wavefronts until the final merge. Chunks travel
// HBM -> LDS with global_load_lds_dwordx4 (no registers, no ds_write); chunk c + A4_SLOTS is issued as
// soon as chunk c has been read.
//
// A record is 2 D / 64 chunks (eight at D = 256): the K payload of channel tiles 4s .. 4s+3 (s < D / 64) for
// all 8 token tiles, then the V payload in the same cut (channel tiles 4J .. 4J+3); a chunk holds its 32 tiles
// as [token tile][channel tile - 4s] x 128 B. The scales travel in two small buffers per wavefront. At
// D = 256 they are issued as soon as the previous record no longer reads them: Kscale | Kzero | Ktok (1280 B,
// after the record's softmax) and Vch | Vscale | Vzero (1024 B, after its last V chunk) (sj_kvarn.h:771-790);
// at D = 128 (768 B each) they are double-buffered, as described below.
//
// QK: lane (n, g) reads 16 bytes of K tile (token tile 2p + n/8, channel tile 4s + g), fragment words
// 4(n&7) .. +3, i.e. tokens t0 = 16(2p + n/8) + n%8 and t0 + 8 x all 16 channels of the tile
// (sj_kvarn.h:807-833). The masks 0x000F000F / 0x00F000F0, on the words and on their 8-bit rotations,
// give four MFMA A operands (token t0 or t0 + 8, channels 0-7 or 8-15) of codes x 2^-24 or x 2^-20;
// Q' = Q * Kscale (fp16 hi + lo) is the B operand. Scores of token tile pair p land as S^T: lane (n, g)
// holds query n, tokens 32p + tb(g) + i and + 8 + i (i < 4, tb(g) = 16(g/2) + 4(g&1)), which is exactly
// the A operand (k = 8 tokens) of the PV product for query n, so P' never leaves the lane.
//
// PV: lane (n, g) reads 8 bytes of V tile (token tile 2p + g/2, channel tile 2J + n/8), words
// 4(n&7) + 2(g&1) .. +1: channel c0 = 16(2J + n/8) + n%8 and c0 + 8 x the lane group's 8 tokens.
// O tile 2J + m (m = 0: channel c0, m = 1: c0 + 8) is column n of lane (n, g), rows 4g + i.

// Head dimension 128: a record is four chunks (K, K, V, V), too few for the scale blocks of the next record to
// be issued behind the chunks of this one and still arrive before they are read. Each wavefront then keeps two
// sets of scale buffers, record i using set i & 1, and issues both blocks of record i + 1 right after its first
// refill in record i (behind chunk 4i + 3, ahead of chunk 4i + 4), into the set record i - 1 has finished with.
constexpr int A4_SLOTS = 3;
constexpr int A4_CHUNK = 4096;
template <int D> struct A4Geom {
    using RL = RecLay4<D>;
    static constexpr int NS = D / 64;                          // 4 KB chunks per side of a record
    static constexpr int CPR = 2 * NS;                         // chunks per record
    static constexpr int TT = D / 16;                          // 16 x 16 tiles per token tile
    static constexpr int KMETA = RL::KTOK + 256 - RL::KSC;     // Kscale | Kzero | Ktok
    static constexpr int VMETA = RL::BYTES - RL::VCH;          // Vch | Vscale | Vzero
    static constexpr int M_KSC = 0, M_KZE = 2 * D, M_KTOK = 4 * D, M_VCH = 0, M_VSC = 2 * D, M_VZE = 2 * D + 256;
    static constexpr int KM_I = (KMETA + 1023) / 1024;         // DMA instructions of a K scale block (16 B a lane)
    static constexpr int VM_I = (VMETA + 1023) / 1024;
    static constexpr int NMETA = D == 256 ? 1 : 2;             // scale buffer sets per wavefront
    static_assert(D == 128 || D == 256, "head dimension of the 4/4 streaming kernel");
    static_assert(RL::KZE - RL::KSC == M_KZE && RL::KTOK - RL::KSC == M_KTOK && RL::VSC - RL::VCH == M_VSC &&
                  RL::VZE - RL::VCH == M_VZE && RL::VCH == RL::KTOK + 256 && RL::KSC % 16 == 0 && RL::VCH % 16 == 0 &&
                  KMETA % 16 == 0 && VMETA % 16 == 0 && VM_I == 1, "scale blocks of a 4/4 record");
};
static_assert(A4Geom<256>::KMETA == 1280 && A4Geom<256>::VMETA == 1024 && A4Geom<256>::KM_I == 2 &&
              A4Geom<128>::KMETA == 768 && A4Geom<128>::VMETA == 768 && A4Geom<128>::KM_I == 1, "scale block sizes");

constexpr int A4_NW = 8;                         // wavefronts per workgroup (two per SIMD)
constexpr int A4_NT = 64 * A4_NW;

// a wavefront's own 16 KB: its stream buffers, then (once its stream is done) its O tiles for the merge
template <int D> struct Rec4Wave {
    using GM = A4Geom<D>;
    uint8_t ring[A4_SLOTS][A4_CHUNK];
    uint8_t kmeta[GM::NMETA][GM::KMETA];
    uint8_t vmeta[GM::NMETA][GM::VMETA];
    uint8_t pad[16384 - A4_SLOTS * A4_CHUNK - GM::NMETA * (GM::KMETA + GM::VMETA)];
};
static_assert(sizeof(Rec4Wave<256>) == 16384 && sizeof(Rec4Wave<128>) == 16384, "16 KB per wavefront: the O tiles of the merge");
template <int D> struct Rec4Lds {
    alignas(16) Rec4Wave<D> wv[A4_NW];
    alignas(16) float q[A3_Q][D + 4];            // query rows (row stride 4 D + 16 B: the lanes of a column spread over the banks)
};
template <int D> using A4Lds = A3LdsT<Rec4Lds<D>, A4_NW>;
static_assert(sizeof(A4Lds<256>) <= 160 * 1024 && sizeof(A4Lds<128>) <= 160 * 1024, "LDS of one workgroup per CU");
static_assert(sizeof(RowLdsT<A4_NW>) <= A4_NW * 16 * 1024, "the row path's merge needs 16 KB per wavefront");

#define SJK_LDS(p) ((__attribute__((address_space(3))) void *) (p))

// cache policy of the stream's loads: non-temporal (every byte is read once per call)
constexpr int A4_POL = 2;

// wait until at most N of this wavefront's vector memory instructions are outstanding (they complete in
// issue order); "memory" keeps the LDS reads after it
template <int N> SJK_DEV void vm_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// all LDS reads issued so far have returned (before a buffer is refilled)
SJK_DEV void lds_reads_done() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 16 floats of LDS (16-byte aligned) read by inline asm, and the wait that makes them usable. The query rows
// arrive by LDS DMA; a compiler-visible read of them makes the compiler wait for every load in flight.
SJK_DEV void lds_read16(const float * p, f4 & x0, f4 & x1, f4 & x2, f4 & x3) {
    const uint32_t ad = (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) float *) p;
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\tds_read_b128 %2, %4 offset:32\n\t"
                 "ds_read_b128 %3, %4 offset:48"
                 : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3) : "v"(ad) : "memory");
}
SJK_DEV void lds_reads_done(f4 & x0, f4 & x1, f4 & x2, f4 & x3) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3) :: "memory");
}

template <int D>
__device__ __attribute__((always_inline)) inline void a4_records(const A3Args & a, A4Lds<D> & S, int h, int wgi, int ls) {
    using GM = A4Geom<D>;
    using RL = typename GM::RL;
    constexpr int NS = GM::NS, CPR = GM::CPR;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const sjk_hip_view & V = a.v;
    const int H = V.n_head_kv;
    // this wavefront's records [r0, r1) of the head: rec_a per wavefront, in slot order (every wavefront but
    // those at the end has the same number, so that every SIMD, whichever two wavefronts it holds, has the same)
    const int per = a.rec_a;
    const int base = (ls * A4_NW + w) * per;
    const int r0 = __builtin_amdgcn_readfirstlane(base < a.n_rec ? base : a.n_rec);
    const int r1 = __builtin_amdgcn_readfirstlane(base + per < a.n_rec ? base + per : a.n_rec);
    const int nrec = r1 - r0, C = CPR * nrec;
    uint8_t * ring = S.r.wv[w].ring[0];
    // the block table is read through the constant address space, i.e. by a scalar load: a vector load
    // would have to wait for every load in flight (the compiler cannot order it against the stream)
    const __attribute__((address_space(4))) uint32_t * blocks = (const __attribute__((address_space(4))) uint32_t *) V.blocks;
    auto rec_base = [&](int r) {
        const uint32_t gi = (a.sink_end + (uint32_t) r * 128u - V.S) / 128u;
        const uint32_t blk = blocks ? blocks[gi] : gi;
        return V.body + ((size_t) blk * H + h) * RL::BYTES;
    };
    auto dma = [&](const uint8_t * src, uint8_t * dst) {
        __builtin_amdgcn_global_load_lds((const void *) src, SJK_LDS(dst), 16, 0, A4_POL);
    };
    // scale buffer set k (k = 0 at D = 256)
    auto kmeta_of = [&](int k) { return S.r.wv[w].kmeta[GM::NMETA == 1 ? 0 : k]; };
    auto vmeta_of = [&](int k) { return S.r.wv[w].vmeta[GM::NMETA == 1 ? 0 : k]; };
    auto issue_kmeta = [&](const uint8_t * rb, int k) {             // KM_I instructions
        uint8_t * km = kmeta_of(k);
        if constexpr (GM::KMETA >= 1024) {
            dma(rb + RL::KSC + 16 * lane, km);
            if (lane < (GM::KMETA - 1024) / 16) dma(rb + RL::KSC + 1024 + 16 * lane, km + 1024);
        } else {
            if (lane < GM::KMETA / 16) dma(rb + RL::KSC + 16 * lane, km);
        }
    };
    auto issue_vmeta = [&](const uint8_t * rb, int k) {             // 1 instruction
        uint8_t * vm = vmeta_of(k);
        if constexpr (GM::VMETA == 1024) dma(rb + RL::VCH + 16 * lane, vm);
        else if (lane < GM::VMETA / 16) dma(rb + RL::VCH + 16 * lane, vm);
    };
    // chunk c (unit u = c % CPR of record c / CPR), 4 instructions: lane l of instruction k4 moves 16 bytes
    // of tile (token tile 2 k4 + l/32, channel tile 4(u % NS) + (l/8 & 3)) into slot byte 1024 k4 + 16 l
    auto issue_chunk = [&](const uint8_t * rb, int c) {
        const int u = c % CPR;
        const uint8_t * src = rb + (u < NS ? 0 : RL::VPAY) +
                              (GM::TT * (lane >> 5) + 4 * (u % NS) + ((lane >> 3) & 3)) * 128 + 16 * (lane & 7);
        uint8_t * dst = ring + (c % A4_SLOTS) * A4_CHUNK;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) dma(src + 2 * k4 * GM::TT * 128, dst + 1024 * k4);
    };

    // Q rows: wavefront w moves rows 2w, 2w + 1 (one instruction each, 4 D bytes to the row of the LDS copy),
    // then the stream starts: the scales of record 0 and its first chunk
    static_assert(A3_Q == 2 * A4_NW, "two query rows per wavefront");
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
        if (D == 256 || lane < D / 4)
            __builtin_amdgcn_global_load_lds((const void *) (q_row<D>(a, h, 2 * w + k2) + 4 * lane),
                                             SJK_LDS(&S.r.q[2 * w + k2][0]), 16, 0, 0);
    // Only chunk 0 goes out with the scales before the barrier: every wavefront's first chunk then comes
    // ahead of the second and third chunks of all the others (the start is a burst of all wavefronts).
    const uint8_t * rb_cur = nullptr;
    if (nrec > 0) {
        rb_cur = rec_base(r0);
        issue_kmeta(rb_cur, 0);
        issue_vmeta(rb_cur, 0);
        issue_chunk(rb_cur, 0);
        vm_wait<GM::KM_I + GM::VM_I + 4>();     // this wavefront's Q rows have arrived (issued before these)
    } else {
        vm_wait<0>();
    }
    // every wavefront's Q rows are in (each waited for its own above); a bare s_barrier: __syncthreads()
    // would also wait for the stream's first chunks
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (nrec > 0) {
#pragma unroll
        for (int c = 1; c < A4_SLOTS; ++c) issue_chunk(rb_cur, c);
    }

    float m_run = -__builtin_inff(), l_run = 0.0f;
    constexpr int NJ = D / 16;                   // O tiles
    f4 O[NJ];                                    // O tile 2J + m: column n = channel 32J + 16(n>>3) + (n&7) + 8m
#pragma unroll
    for (int j = 0; j < NJ; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t qend = q_end(a, n);
    const uint32_t qend_min = q_end(a, 0);       // q_end grows with the row over the live rows
    const int tbg = 16 * (g >> 1) + 4 * (g & 1); // first score token of the lane group in a 32-token step
    const uint32_t M0 = 0x000F000Fu, M1 = 0x00F000F0u;
    const float * qlane = &S.r.q[n][0];

    const uint8_t * rb_next = (nrec > 1) ? rec_base(r0 + 1) : nullptr;
    for (int i = 0; i < nrec; ++i) {
        const bool last = i + 1 == nrec;
        const uint8_t * rb_after = (i + 2 < nrec) ? rec_base(r0 + i + 2) : nullptr;
        const uint32_t p0 = a.sink_end + (uint32_t) (r0 + i) * 128u;
        const int mb = GM::NMETA == 1 ? 0 : (i & 1);              // this record's scale buffer set
        const uint8_t * kmeta = kmeta_of(mb);
        const uint8_t * vmeta = vmeta_of(mb);
        // vmcnt while waiting for chunk CPR i + u: the loads issued after it may still be in flight.
        // D = 256: the next two chunks, plus the K scales of record i + 1 (u = 4, 5, 6) or the V scales of
        // record i (u = 0, 1, 2 after the first record, not counted: a wait that is one short only waits
        // longer). D = 128: the next two chunks, plus both scale blocks of record i + 1 (u = 1, 2, 3; issued
        // behind chunk 4i + 3). The last record issues nothing past its own chunks.
        auto wait_unit = [&](int u) {
            if constexpr (D == 256) {
                if (!last) {
                    if (u >= 4 && u <= 6) vm_wait<10>();
                    else vm_wait<8>();
                } else {
                    if (u <= 5) vm_wait<8>();
                    else if (u == 6) vm_wait<4>();
                    else vm_wait<0>();
                }
            } else {
                if (!last) {
                    if (u == 0) vm_wait<8>();
                    else vm_wait<8 + GM::KM_I + GM::VM_I>();
                } else {
                    if (u <= 1) vm_wait<8>();
                    else if (u == 2) vm_wait<4>();
                    else vm_wait<0>();
                }
            }
        };
        auto refill = [&](int c) {               // after chunk c has been read
            if (c + A4_SLOTS < C) issue_chunk((c + A4_SLOTS) / CPR == i ? rb_cur : rb_next, c + A4_SLOTS);
        };

        // ---- QK, one chunk of 64 channels at a time ----
        f4 sl[4], sh[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) { sl[p] = f4{0.0f, 0.0f, 0.0f, 0.0f}; sh[p] = sl[p]; }
        float corr = 0.0f;                       // sum_d Q * Kzero over the lane's channels
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int c = CPR * i + s;
            if (s == 0) prio_by_progress(c, C);
            wait_unit(s);
            const uint8_t * ck = ring + (c % A4_SLOTS) * A4_CHUNK + ((n >> 3) * 4 + g) * 128 + 16 * (n & 7);
            u4 kw[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) kw[p] = *(const u4 *) (ck + p * 8 * 128);
            // Kscale index k_ch_idx(d) (sj_kvarn.h:835-841) puts channels 2j, 2j+1, 2j+8, 2j+9 of channel
            // tile cb in one 8-byte run j at (D / 4) j + 4 cb
            u2 ks[4], kz[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t o = 2u * (uint32_t) ((D / 4) * j + 4 * (4 * s + g));
                ks[j] = *(const u2 *) (kmeta + GM::M_KSC + o);
                kz[j] = *(const u2 *) (kmeta + GM::M_KZE + o);
            }
            f4 qv[4];                            // channel 16(4s + g) + 4 j4 + r of query n: qv[j4][r]
            lds_read16(qlane + 16 * (4 * s + g), qv[0], qv[1], qv[2], qv[3]);
            lds_reads_done(qv[0], qv[1], qv[2], qv[3]);
            refill(c);
            // D = 128: both scale blocks of record i + 1, behind chunk 4i + 3, into the set record i - 1 used
            // (its reads have returned: lds_reads_done before the refills of its last chunk)
            if constexpr (GM::NMETA == 2)
                if (s == 0 && !last) {
                    issue_kmeta(rb_next, mb ^ 1);
                    issue_vmeta(rb_next, mb ^ 1);
                }
            float q[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) q[j] = qv[j >> 2][j & 3];
            u4 qxh, qxl, qyh, qyl;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u2 hx = mul_split(q[2 * j], q[2 * j + 1], ks[j].x);
                const u2 hy = mul_split(q[2 * j + 8], q[2 * j + 9], ks[j].y);
                qxh[j] = hx.x; qxl[j] = hx.y;
                qyh[j] = hy.x; qyl[j] = hy.y;
                corr = fma_lo(q[2 * j], kz[j].x, corr);
                corr = fma_hi(q[2 * j + 1], kz[j].x, corr);
                corr = fma_lo(q[2 * j + 8], kz[j].y, corr);
                corr = fma_hi(q[2 * j + 9], kz[j].y, corr);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const u4 w4 = kw[p];
                const u4 rr = u4{w4[0] >> 8, w4[1] >> 8, w4[2] >> 8, w4[3] >> 8};
                const u4 a0 = w4 & M0, a1 = rr & M0, a2 = w4 & M1, a3 = rr & M1;
                sl[p] = mfma32(a0, qxh, sl[p]);
                sh[p] = mfma32(a2, qxh, sh[p]);
                sl[p] = mfma32(a0, qxl, sl[p]);
                sh[p] = mfma32(a2, qxl, sh[p]);
                sl[p] = mfma32(a1, qyh, sl[p]);
                sh[p] = mfma32(a3, qyh, sh[p]);
                sl[p] = mfma32(a1, qyl, sl[p]);
                sh[p] = mfma32(a3, qyl, sh[p]);
            }
        }

        // ---- scores (log2 units) and the online softmax ----
        // S = Ktok * (sum_d Q' c + corr) * scale * log2 e; the code scale (2^24 for the low nibbles, 2^20 for
        // the high ones) is removed by an ordinary fma first: the accumulators are MFMA results, which the
        // asm of mul_lo / mul_hi must not read
        const float cs = rows_sum(corr) * a.sc2;
        const float s24 = a.sc2 * 0x1p24f, s20 = a.sc2 * 0x1p20f;
        float sc[32];                            // [p][tokens tbg + 0..3 | tbg + 8..11]
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u2 ka = *(const u2 *) (kmeta + GM::M_KTOK + 2 * (32 * p + tbg));
            const u2 kb = *(const u2 *) (kmeta + GM::M_KTOK + 2 * (32 * p + tbg + 8));
            f4 xl, xh;
#pragma unroll
            for (int r = 0; r < 4; ++r) { xl[r] = __builtin_fmaf(sl[p][r], s24, cs); xh[r] = __builtin_fmaf(sh[p][r], s20, cs); }
            sc[8 * p + 0] = mul_lo(xl[0], ka.x);
            sc[8 * p + 1] = mul_hi(xl[1], ka.x);
            sc[8 * p + 2] = mul_lo(xl[2], ka.y);
            sc[8 * p + 3] = mul_hi(xl[3], ka.y);
            sc[8 * p + 4] = mul_lo(xh[0], kb.x);
            sc[8 * p + 5] = mul_hi(xh[1], kb.x);
            sc[8 * p + 6] = mul_lo(xh[2], kb.y);
            sc[8 * p + 7] = mul_hi(xh[3], kb.y);
        }
        if (p0 + 128u > qend_min) {
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const uint32_t tok = (uint32_t) (32 * (e >> 3) + tbg + (e & 3) + 8 * ((e >> 2) & 1));
                if (p0 + tok >= qend) sc[e] = -__builtin_inff();
            }
        }
        // P' = P * Vscale * 2^k with max Vscale in [2^(e-1), 2^e), k = 14 - e: below 2^14, and the small
        // weights stay clear of the fp16 subnormal range
        int kx;
        {
            const uint32_t wv = *(const uint32_t *) (vmeta + GM::M_VSC + 4 * lane);
            const uint32_t mx = wave_umax(max(wv & 0xFFFFu, wv >> 16));   // non-negative halves order like their bits
            kx = 14 - __builtin_amdgcn_frexp_expf(h2f(mx));
        }
        const float pinv = __builtin_amdgcn_ldexpf(1.0f, -kx);
        float mloc = sc[0];
#pragma unroll
        for (int e = 1; e < 32; ++e) mloc = fmaxf(mloc, sc[e]);
        mloc = rows_max(mloc);
        const float m_new = fmaxf(m_run, mloc);
        const bool anyv = m_new != -__builtin_inff();
        const float alpha = anyv ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        // exp2(s - mk) = P * 2^k; a row with no visible token has only -inf scores, and exp2(-inf - 0) = 0
        const float mk = anyv ? m_new - (float) kx : 0.0f;
        float psum = 0.0f, cv = 0.0f;
        u4 Ah[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float & x = sc[8 * p + e];
                x = __builtin_amdgcn_exp2f(x - mk);
                psum += x;
            }
            const u2 vs0 = *(const u2 *) (vmeta + GM::M_VSC + 2 * (32 * p + tbg));
            const u2 vs1 = *(const u2 *) (vmeta + GM::M_VSC + 2 * (32 * p + tbg + 8));
            const u2 vz0 = *(const u2 *) (vmeta + GM::M_VZE + 2 * (32 * p + tbg));
            const u2 vz1 = *(const u2 *) (vmeta + GM::M_VZE + 2 * (32 * p + tbg + 8));
            Ah[p] = u4{mul_pk(sc[8 * p + 0], sc[8 * p + 1], vs0.x), mul_pk(sc[8 * p + 2], sc[8 * p + 3], vs0.y),
                       mul_pk(sc[8 * p + 4], sc[8 * p + 5], vs1.x), mul_pk(sc[8 * p + 6], sc[8 * p + 7], vs1.y)};
            cv = fma_lo(sc[8 * p + 0], vz0.x, cv);
            cv = fma_hi(sc[8 * p + 1], vz0.x, cv);
            cv = fma_lo(sc[8 * p + 2], vz0.y, cv);
            cv = fma_hi(sc[8 * p + 3], vz0.y, cv);
            cv = fma_lo(sc[8 * p + 4], vz1.x, cv);
            cv = fma_hi(sc[8 * p + 5], vz1.x, cv);
            cv = fma_lo(sc[8 * p + 6], vz1.y, cv);
            cv = fma_hi(sc[8 * p + 7], vz1.y, cv);
        }
        lds_reads_done();
        if constexpr (GM::NMETA == 1)
            if (!last) issue_kmeta(rb_next, 0);  // the K scales of this record have been read
        psum = rows_sum(psum);
        cv = rows_sum(cv);
        m_run = m_new;
        l_run = l_run * alpha + psum * pinv;
        {   // unconditional: behind a branch the compiler kept O in two register sets (128 moves per record)
            float arow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) arow[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) O[j][r] = O[j][r] * arow[r];
        }
        f4 c0v, c1v;                             // sum_t P' Vzero of rows 4g + r, in the code scale of the tile
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float cr = __shfl(cv, 4 * g + r, 64);
            c0v[r] = cr * 0x1p-24f;
            c1v[r] = cr * 0x1p-20f;
        }

        // ---- PV, one chunk of 64 channels (O tiles 4J2 .. 4J2+3) at a time ----
#pragma unroll
        for (int J2 = 0; J2 < NS; ++J2) {
            const int c = CPR * i + NS + J2;
            if (J2 == 0) prio_by_progress(c, C);
            wait_unit(NS + J2);
            const uint8_t * cvp = ring + (c % A4_SLOTS) * A4_CHUNK + ((g >> 1) * 4 + (n >> 3)) * 128 + 16 * (n & 7) + 8 * (g & 1);
            u2 vw[4][2];
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) vw[p][jj] = *(const u2 *) (cvp + (p * 8 + 2 * jj) * 128);
            // Vch index v_ch_idx(d) (sj_kvarn.h:843-849): channels c0 and c0 + 8 share a dword
            uint32_t vch[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                vch[jj] = *(const uint32_t *) (vmeta + GM::M_VCH + 2 * ((D / 8) * (n & 7) + 4 * (2 * J2 + jj) + 2 * (n >> 3)));
            lds_reads_done();
            refill(c);
            f4 t[4] = {c0v, c1v, c0v, c1v};      // tiles 2J + m, J = 2 J2 + jj: t[2 jj + m]
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const uint32_t w0 = vw[p][jj].x, w1 = vw[p][jj].y, x0 = w0 >> 8, x1 = w1 >> 8;
                    const u4 b0 = u4{w0 & M0, w1 & M0, x0 & M0, x1 & M0};
                    const u4 b1 = u4{w0 & M1, w1 & M1, x0 & M1, x1 & M1};
                    t[2 * jj] = mfma32(Ah[p], b0, t[2 * jj]);
                    t[2 * jj + 1] = mfma32(Ah[p], b1, t[2 * jj + 1]);
                }
            // O += Vch * 2^-k * t
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int J = 2 * J2 + jj;
                const float v0 = h2f(vch[jj] & 0xFFFFu) * pinv * 0x1p24f, v1 = h2f(vch[jj] >> 16) * pinv * 0x1p20f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    O[2 * J][r] = __builtin_fmaf(v0, t[2 * jj][r], O[2 * J][r]);
                    O[2 * J + 1][r] = __builtin_fmaf(v1, t[2 * jj + 1][r], O[2 * J + 1][r]);
                }
            }
        }
        if constexpr (GM::NMETA == 1)
            if (!last) issue_vmeta(rb_next, 0);  // the V scales of this record have been read (lgkmcnt above)
        rb_cur = rb_next;
        rb_next = rb_after;
    }
    // the stream is done (its last wait was vmcnt(0)) and its LDS reads have returned: the wavefront's O
    // tiles go to its own area while the others still run. O tile j = 2J + m, column n holds channel
    // 32J + 16(n>>3) + (n&7) + 8m.
    lds_reads_done();
    partial_put<NJ>(S, (f4 *) &S.r.wv[w], O, m_run, l_run);
    partial_gather<D>(a, S, (const f4 *) &S.r.wv[0], (int) (sizeof(Rec4Wave<D>) / sizeof(f4)), h, wgi, [](int d, int & j, int & nn) {
        j = 2 * (d >> 5) + ((d >> 3) & 1);
        nn = 8 * ((d >> 4) & 1) + (d & 7);
    });
}

// ------------------------------------------------------------------------------------------------
// trellis record workgroups
// ------------------------------------------------------------------------------------------------

template <int BK, int BV, int D, typename Lds>
__device__ __attribute__((always_inline)) inline void a3_trellis(const A3Args & a, Lds & S, int h, int wgi, int r0, int r1) {
    static_assert(D == 128 || D == 256, "head dimension of the trellis kernel");
    constexpr int CPT = D / 16;                  // channels per Q' builder thread
    constexpr int NJW = D / 64;                  // PV channel tiles per wavefront
    using RL = RecLay<BK, BV, D>;
    auto & s = S.r;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    const sjk_hip_view & V = a.v;
    const int H = V.n_head_kv;
    // the first record's loads go out before anything else
    constexpr int NV = RL::BYTES / 16, PF = (NV + A3_NT - 1) / A3_NT;
    u4 pf[PF];
    auto fetch = [&](int c) {
        const uint32_t gi = (a.sink_end + (uint32_t) c * 128u - V.S) / 128u;
        const uint32_t blk = V.blocks ? V.blocks[gi] : gi;
        const u4 * src = (const u4 *) (V.body + ((size_t) blk * H + h) * RL::BYTES);
#pragma unroll
        for (int k = 0; k < PF; ++k)
            if (tid + A3_NT * k < NV) pf[k] = src[tid + A3_NT * k];
    };
    if (r0 < r1) fetch(r0);
    // byte-offset masks of the pair tables (index << 2)
    constexpr uint32_t KM4 = ((1u << (6 + 2 * BK)) - 1u) << 2, VM4 = ((1u << (6 + 2 * BV)) - 1u) << 2;
    {
        // all loads of both tables issued before the first store (one round trip)
        constexpr int NK = (1 << (6 + 2 * BK)) / 4 / A3_NT, NVT = (1 << (6 + 2 * BV)) / 4 / A3_NT;
        static_assert(NK >= 1 && NVT >= 1, "pair tables of at least one u4 per thread");
        const u4 * tk = (const u4 *) pair_tab<BK, false>();
        const u4 * tv = (const u4 *) pair_tab<BV, true>();
        u4 bk[NK], bvv[NVT];
#pragma unroll
        for (int k = 0; k < NK; ++k) bk[k] = tk[tid + A3_NT * k];
#pragma unroll
        for (int k = 0; k < NVT; ++k) bvv[k] = tv[tid + A3_NT * k];
#pragma unroll
        for (int k = 0; k < NK; ++k) ((u4 *) s.tk)[tid + A3_NT * k] = bk[k];
#pragma unroll
        for (int k = 0; k < NVT; ++k) ((u4 *) s.tv)[tid + A3_NT * k] = bvv[k];
        if (tid < 4) s.zero[tid] = 0u;
        // the dword after each channel stream (the one read before the next channel's start) stays zero: staging
        // writes only stream bytes, so the lanes whose window starts before the stream need no mask
        static_assert(A3_NT >= D, "one K and one V channel per thread");
        using P = TrPad<BK, BV, D>;
        if (tid < D) {
            *(uint32_t *) (s.rec + P::KSTR * tid + 16 * BK) = 0u;
            *(uint32_t *) (s.rec + P::VPAY + P::VSTR * tid + 16 * BV) = 0u;
        }
    }
    // Q' builder role: thread (query bq, CPT-channel block bc); B-operand slot (k-step ks, lane group gg,
    // slot i) is channel 32 ks + 8 gg + i
    const int bq = tid & 15, bc = tid >> 4;
    float qv[CPT];
    {
        const float * qr = q_row<D>(a, h, bq) + CPT * bc;
        const bool live = bq < a.n_rows;
#pragma unroll
        for (int k = 0; k < CPT; k += 4) {
            const float4 x4 = *(const float4 *) (qr + k);
            qv[k] = live ? x4.x : 0.0f; qv[k + 1] = live ? x4.y : 0.0f;
            qv[k + 2] = live ? x4.z : 0.0f; qv[k + 3] = live ? x4.w : 0.0f;
        }
    }
    const uint32_t qend = q_end(a, n);
    const uint32_t qend_min = q_end(a, 0);       // q_end grows with the row over the live rows
    // Stream words: bit j of x = alignbit(hi, lo, sh) is stream bit r + j of the channel, r = (first
    // token) * bits - 8, so that x & mask is the table byte offset of the pair starting at that token
    // (6 history bits from r + 2 on). Stream bits before the channel start are zero: lanes with r < 0
    // read the dword before the stream as lo and clear it.
    // K: tokens 32w + 2n and +1 (QK row n of tiles 0 and 1), channels 32 ks + 8 g + i
    const int kr = BK * (32 * w + 2 * n) - 8;
    const uint32_t ksh = (uint32_t) (kr + 32) & 31u;
    using P = TrPad<BK, BV, D>;
    // stream words of k-step ks: one base address per k-step (kept opaque, so that the eight channels' reads
    // take their offsets as instruction immediates instead of one address add each)
    const uint32_t kofs = (uint32_t) (4 * (((kr + 32) >> 5) - 1) + P::KSTR * 8 * g);
    auto kp_base = [&](int ks) {
        uint32_t o = kofs + (uint32_t) (P::KSTR * 32 * ks);
        asm volatile("" : "+v"(o));
        return s.rec + o;
    };
    // V of k-step m (the tokens of wave m): tokens 32m + 8g .. +7 (the PV k-slots of lane group g),
    // channel 16 J + n of this wave's channel tiles J = NJW w + jj
    // (stream bit r = vr0 + 32 BV m, m = k-step: the same word offset within a dword for every m)
    const int vr0 = BV * (8 * g) - 8;                                // k-step 0: r < 0 for g = 0
    const uint32_t vsh = (uint32_t) (vr0 + 32) & 31u;
    const uint32_t vofs = (uint32_t) (P::VPAY + P::VSTR * (n + (D / 4) * w) + 4 * (((vr0 + 32) >> 5) - 1));
    const int tok0 = 32 * w + 8 * g;                                 // the lane's 8 score tokens

    float m_run = -__builtin_inff(), l_run = 0.0f;                  // m shared by the waves, l over own tokens
    f4 O[NJW];                                                       // channel tile NJW w + jj
#pragma unroll
    for (int j = 0; j < NJW; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};


    for (int c = r0; c < r1; ++c) {
        prio_by_progress(c - r0, r1 - r0);
        const uint32_t p0 = a.sink_end + (uint32_t) c * 128u;
        __syncthreads();
        {
            // 16 bytes of the record per thread and step, to their place in the padded layout (a 16-byte piece never
            // straddles two channel streams: they are 48 or 32 bytes)
#pragma unroll
            for (int k = 0; k < PF; ++k) {
                const int kk = tid + A3_NT * k;
                if (kk >= NV) continue;
                const int o = 16 * kk;
                if (o >= RL::KSC) {
                    *(u4 *) (s.rec + P::KSC + (o - RL::KSC)) = pf[k];
                } else {
                    const bool v = o >= RL::VPAY;
                    const int o2 = v ? o - RL::VPAY : o, cb = v ? 16 * BV : 16 * BK, ch = o2 / cb;
                    uint32_t * d = (uint32_t *) (s.rec + (v ? P::VPAY + ch * P::VSTR : ch * P::KSTR) + (o2 - ch * cb));
                    d[0] = pf[k].x; d[1] = pf[k].y; d[2] = pf[k].z; d[3] = pf[k].w;
                }
            }
        }
        if (c + 1 < r1) fetch(c + 1);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // Q' = Q * Kscale (hi / lo) and this thread's part of sum_d Q * Kzero (Kscale index = channel)
        {
            float corr = 0.0f;
#pragma unroll
            for (int e = 0; e < CPT / 8; ++e) {
                const int ch0 = CPT * bc + 8 * e;                   // channels ch0 .. ch0 + 7
                const u4 ks = *(const u4 *) (s.rec + P::KSC + 2 * ch0);
                const u4 kz = *(const u4 *) (s.rec + P::KZE + 2 * ch0);
                u4 hi, lo;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int c0 = 8 * e + 2 * u;
                    corr = fma_lo(qv[c0], kz[u], corr);
                    corr = fma_hi(qv[c0 + 1], kz[u], corr);
                    const u2 hl = mul_split(qv[c0], qv[c0 + 1], ks[u]);
                    hi[u] = hl.x;
                    lo[u] = hl.y;
                }
                const int kss = ch0 >> 5, gg = (ch0 >> 3) & 3;
                *(u4 *) &s.op.qb[0][kss][gg][bq][0] = hi;
                *(u4 *) &s.op.qb[1][kss][gg][bq][0] = lo;
            }
            corr = rows_sum(corr);
            if (g == 0) s.corr[w][bq] = corr;
        }
        __syncthreads();
        f4 acc[2], acl[2];
        {
            const float ck = (s.corr[0][n] + s.corr[1][n]) + (s.corr[2][n] + s.corr[3][n]);
            acc[0] = f4{ck, ck, ck, ck};
            acc[1] = acc[0];
            acl[0] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            acl[1] = acl[0];
        }
        // two k-steps (16 channels) at a time: all stream words, then all pair lookups, then the MFMAs, so
        // that each batch waits for LDS twice instead of once per channel
#pragma unroll
        for (int kp = 0; kp < D / 32; kp += 2) {
            uint32_t wl[16], wh[16], L[16];  // channel 32 ks + 8 g + i (ks = kp + (k >> 3), i = k & 7)
            const uint8_t * kb[2] = {kp_base(kp), kp_base(kp + 1)};
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const uint8_t * q = kb[k >> 3] + P::KSTR * (k & 7);
                wl[k] = *(const uint32_t *) q;
                wh[k] = *(const uint32_t *) (q + 4);
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const uint32_t x = __builtin_amdgcn_alignbit(wh[k], wl[k], ksh);
                L[k] = *(const uint32_t *) ((const uint8_t *) s.tk + (x & KM4));
            }
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int ks = kp + h2;
                const u4 Bh = *(const u4 *) &s.op.qb[0][ks][g][n][0];
                const u4 Bl = *(const u4 *) &s.op.qb[1][ks][g][n][0];
                u4 A0, A1;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    A0[u] = __builtin_amdgcn_perm(L[8 * h2 + 2 * u + 1], L[8 * h2 + 2 * u], 0x05040100u);
                    A1[u] = __builtin_amdgcn_perm(L[8 * h2 + 2 * u + 1], L[8 * h2 + 2 * u], 0x07060302u);
                }
                acc[0] = mfma32(A0, Bh, acc[0]);
                acl[0] = mfma32(A0, Bl, acl[0]);
                acc[1] = mfma32(A1, Bh, acc[1]);
                acl[1] = mfma32(A1, Bl, acl[1]);
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[tt] = acc[tt] + acl[tt];
        // C row 4g + i of tile tt is token 32w + 8g + 2i + tt: score k = 2i + tt is token tok0 + k
        float sc[8];
        {
            const u4 kt = *(const u4 *) (s.rec + P::KTOK + 2 * tok0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[2 * i] = mul_lo(acc[0][i], kt[i]) * a.sc2;
                sc[2 * i + 1] = mul_hi(acc[1][i], kt[i]) * a.sc2;
            }
        }
        if (p0 + 128u > qend_min) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (p0 + (uint32_t) (tok0 + k) >= qend) sc[k] = -__builtin_inff();
        }
        // the record's maximum per query, agreed by the four waves
        float mloc = sc[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) mloc = fmaxf(mloc, sc[k]);
        mloc = rows_max(mloc);
        if (g == 0) s.wmax[w][n] = mloc;
        __syncthreads();
        const float m_new = fmaxf(m_run, fmaxf(fmaxf(s.wmax[0][n], s.wmax[1][n]), fmaxf(s.wmax[2][n], s.wmax[3][n])));
        const bool anyv = m_new != -__builtin_inff();
        const float alpha = anyv ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        float psum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            sc[k] = anyv ? __builtin_amdgcn_exp2f(sc[k] - m_new) : 0.0f;
            psum += sc[k];
        }
        psum = rows_sum(psum);
        m_run = m_new;
        l_run = l_run * alpha + psum;
        // P' = P * Vscale * 2^k (fp16): A-operand slot k of k-step w = token tok0 + k; corrV = sum_t P * Vzero
        // (scaled alike)
        float pinv;
        const float psc = pv_scale(s.rec + P::VSC, lane, pinv);
#pragma unroll
        for (int k = 0; k < 8; ++k) sc[k] = sc[k] * psc;
        {
            u4 Ah;
            float cv = 0.0f;
            const u4 vs = *(const u4 *) (s.rec + P::VSC + 2 * tok0);
            const u4 vz = *(const u4 *) (s.rec + P::VZE + 2 * tok0);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                Ah[u] = mul_pk(sc[2 * u], sc[2 * u + 1], vs[u]);
                cv = fma_lo(sc[2 * u], vz[u], cv);
                cv = fma_hi(sc[2 * u + 1], vz[u], cv);
            }
            cv = rows_sum(cv);
            s.op.pa[w][lane] = Ah;
            if (g == 0) s.cvp[w][n] = cv;
        }
        float arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * g + i, 64);
        if (__any(arow[0] != 1.0f || arow[1] != 1.0f || arow[2] != 1.0f || arow[3] != 1.0f)) {
#pragma unroll
            for (int j = 0; j < NJW; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) O[j][i] = O[j][i] * arow[i];
        }
        uint32_t vchw[NJW];
#pragma unroll
        for (int jj = 0; jj < NJW; ++jj) vchw[jj] = *(const uint16_t *) (s.rec + P::VCH + 2 * (16 * (NJW * w + jj) + n));
        __syncthreads();
        u4 Ah[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) Ah[m] = s.op.pa[m][lane];
        f4 crow;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = 4 * g + i;
            crow[i] = (s.cvp[0][q] + s.cvp[1][q]) + (s.cvp[2][q] + s.cvp[3][q]);
        }
        // PV tile J = NJW w + jj: column n = channel 16 J + n; k-step m: the four pair lookups of tokens
        // 32m + 8g .. +7 are the B operand as they stand
#pragma unroll
        for (int jj = 0; jj < NJW; ++jj) {
            f4 t = crow;
            uint32_t vo = vofs + (uint32_t) (16 * P::VSTR * jj);
            asm volatile("" : "+v"(vo));
            const uint8_t * vb = s.rec + vo;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint8_t * q = vb + 4 * BV * m;                 // stream bit origin vr0 + 32 BV m
                const uint32_t x = __builtin_amdgcn_alignbit(*(const uint32_t *) (q + 4), *(const uint32_t *) q, vsh);
                u4 Bv;
#pragma unroll
                for (int u = 0; u < 4; ++u) Bv[u] = *(const uint32_t *) ((const uint8_t *) s.tv + ((x >> (2 * BV * u)) & VM4));
                t = mfma32(Ah[m], Bv, t);
            }
            const float vc = h2f(vchw[jj]) * pinv;
#pragma unroll
            for (int i = 0; i < 4; ++i) O[jj][i] = __builtin_fmaf(vc, t[i], O[jj][i]);
        }
    }
    write_partial_cs<D>(a, S, h, wgi, O, m_run, l_run, 1.0f);
}

// ------------------------------------------------------------------------------------------------
// row workgroups (sink and staging tail)
// ------------------------------------------------------------------------------------------------

// dword at a 2-byte-aligned LDS address
SJK_DEV uint32_t lds_u32_a2(const uint8_t * p) {
    return (uint32_t) *(const uint16_t *) p | ((uint32_t) *(const uint16_t *) (p + 2) << 16);
}

// tq6_0 pair table: two neighbouring channels 2u, 2u+1 of a block share qs byte u (their low nibbles) and qh
// nibble u (their high bit pairs), sj_kvarn.h:1255-1257. Entry (qs byte | qh nibble << 8) holds the two
// centroids as fp16 {hi pair, lo pair}, i.e. two MFMA operand dwords.
SJK_DEV void tq6_pair_entry(uint32_t e, const float * cent, u2 & out) {
    const int c0 = (int) ((e & 15u) | (((e >> 8) & 3u) << 4));
    const int c1 = (int) (((e >> 4) & 15u) | (((e >> 10) & 3u) << 4));
    out = split2(cent[c0], cent[c1]);
}

// 8 tq6_0 values (channels 8 c8 .. 8 c8 + 7 of a 128-value block; centroids, without the block norm) as fp16
// hi and lo pairs, one pair-table lookup per two channels: pair u holds channels 2u, 2u+1
SJK_DEV void tq6_pairs8(const uint8_t * blk, int c8, const u2 * pt, u4 & vh, u4 & vl) {
    const uint32_t qs = lds_u32_a2(blk + 2 + 4 * c8);
    const uint32_t qh = *(const uint16_t *) (blk + 66 + 2 * c8);
    const uint32_t b = __builtin_amdgcn_perm(qh, qh, 0x01010000u);        // bytes [qh0, qh0, qh1, qh1]
    const uint32_t z = (b & 0x000F000Fu) | ((b >> 4) & 0x0F000F00u);       // byte u = qh nibble u
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        // [qs byte u, z byte u, 0, 0]
        const uint32_t idx = __builtin_amdgcn_perm(z, qs, 0x0C0C0000u | ((uint32_t) (4 + u) << 8) | (uint32_t) u);
        const u2 e = pt[idx];
        vh[u] = e.x;
        vl[u] = e.y;
    }
}

// DEPTH: chunks whose rows are held in registers ahead of the one being computed (the next DEPTH chunks
// of the wavefront are in flight while it computes)
// fin(O, m, l, chan) writes the wavefronts' state as the workgroup's partial (chan(j, n): channel of O tile j,
// column n).
// D: head dimension (128 or 256); NB = D / 128 tq6_0 blocks per row, O tiles 8 NB.
template <int DEPTH, int D, typename Lds, typename Fin>
__device__ __attribute__((always_inline)) inline void a3_rows(const A3Args & a, Lds & S, int h, int wgr, Fin fin) {
    static_assert(D == 128 || D == 256, "head dimension of the row path");
    constexpr int NB = D / 128;
    auto & s = S.w;
    constexpr int NW = sizeof(s.stage) / sizeof(s.stage[0]);     // wavefronts of the workgroup
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    const sjk_hip_view & V = a.v;
    const uint32_t qend = q_end(a, n);
    float m_run = -__builtin_inff(), l_run = 0.0f;
    f4 O[8 * NB];
#pragma unroll
    for (int j = 0; j < 8 * NB; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int wu = __builtin_amdgcn_readfirstlane(w);
    uint8_t * st = s.stage[wu];
    const int waves = NW * a.n_row_wg;
    // the job and view fields of the loop, in registers that the compiler cannot re-load: at the register
    // budget of this kernel it would otherwise re-read them from the kernel arguments in every step, each a
    // round trip of its own
    int r_sinkc = a.sink_chunks, r_nch = a.n_chunk;
    uint32_t r_bend = a.body_end, r_send = a.sink_end, r_pend = a.pend, r_S = V.S, r_cap = V.cap;
    uint32_t r_H = (uint32_t) V.n_head_kv, r_vo = (uint32_t) V.stage_bytes;
    uint32_t r_f16 = (V.sink_type == SJKVARN_SINK_F16 ? 1u : 0u) | (V.staging == SJKVARN_STAGING_F16 ? 2u : 0u);
    typedef const __attribute__((address_space(1))) uint8_t * gptr;
    gptr r_sink = (gptr) V.sink;
    gptr r_ring = (gptr) V.ring;
    float r_sc2 = a.sc2;
    r_f16 = __builtin_amdgcn_readfirstlane(r_f16);
    r_sc2 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, r_sc2)));
    asm volatile("" : "+s"(r_sinkc), "+s"(r_nch), "+s"(r_bend), "+s"(r_send), "+s"(r_pend), "+s"(r_S), "+s"(r_cap),
                 "+s"(r_H), "+s"(r_vo), "+s"(r_f16), "+s"(r_sink), "+s"(r_ring), "+s"(r_sc2));
    // K | V row of position p of the head: fp16 sink, inherited sink, or the ring
    auto row_of = [&](uint32_t p) -> gptr {
        if (p < r_S && (r_f16 & 1u)) return r_sink + ((size_t) p * r_H + h) * 4 * D;
        return p < r_S ? r_sink + ((size_t) p * r_H + h) * 2 * r_vo
                       : r_ring + ((size_t) ((p - r_S) % r_cap) * r_H + h) * 2 * r_vo;
    };
    // chunk c: positions [p0, p1) of the sink (c < sink_chunks) or of the tail
    auto chunk = [&](int c, uint32_t & p0, uint32_t & p1) {
        const bool sink = c < r_sinkc;
        p0 = sink ? (uint32_t) (A3_CH * c) : r_bend + (uint32_t) (A3_CH * (c - r_sinkc));
        const uint32_t pe = sink ? r_send : r_pend;
        p1 = p0 + A3_CH < pe ? p0 + A3_CH : pe;
    };
    // tq6_0 rows are staged in the wavefront's LDS slice (K | V, 2 x 98 NB B; fp16 rows are read from HBM
    // where they are used). Lane l < 49 holds word l (2 NB bytes x 4) of each of the 16 rows (rows past p1
    // repeat row p0: finite values, masked below); the row addresses are wave-uniform.
    auto f16_chunk = [&](int c) {
        return (c < r_sinkc && (r_f16 & 1u)) || (r_f16 & 2u);
    };
    typedef typename std::conditional<NB == 2, u2, uint32_t>::type RowWord;
    static_assert(sizeof(RowWord) * 49 == 2 * NB * SJKVARN_TQ6_BLOCK_BYTES, "49 words per K | V row");
    RowWord pfr[DEPTH][A3_CH];
    auto fetch = [&](int c, auto B) {
        constexpr int b = decltype(B)::value;
        if (f16_chunk(c)) return;
        uint32_t p0, p1;
        chunk(c, p0, p1);
        const bool sink = c < r_sinkc;
        const int words = (int) (2 * r_vo / sizeof(RowWord));
        const size_t rs = 2 * (size_t) r_vo;                                   // bytes per (position, head)
        const size_t rowb = (size_t) r_H * rs;                                 // bytes per position
        const gptr base = (sink ? r_sink : r_ring) + (size_t) h * rs;
        const uint32_t slot0 = sink ? p0 : (p0 - r_S) % r_cap;
        const uint32_t nr = p1 - p0;                                          // rows past p1 repeat row p0
        const uint32_t room = sink ? (uint32_t) A3_CH : r_cap - slot0;        // rows before the ring wraps
        const gptr first = base + (size_t) slot0 * rowb;
        // wave-uniform row addresses as a running pointer (slot0 + r, wrapped once: slot0 < cap, 16 <= cap),
        // not recomputed per row (64-bit products, ~27 scalar instructions a row)
        if (lane < words) {
            gptr cur = first;
#pragma unroll
            for (int r = 0; r < A3_CH; ++r) {
                if (r > 0) cur = ((uint32_t) r == room) ? base : cur + rowb;
                const gptr ad = (uint32_t) r < nr ? cur : first;
                pfr[b][r] = *(const __attribute__((address_space(1))) RowWord *) (ad + (uint32_t) (sizeof(RowWord) * lane));
            }
        }
    };
    // chunk c, c + waves, ... of the wave's rank: with 8 waves (two per SIMD: waves w and w + 4), the first
    // waves of all SIMDs rank before the second ones, so that the chunks of a short last round go one per
    // SIMD (a SIMD with two 3-chunk waves ends ~5 us after one with a 3-chunk and a 2-chunk wave)
    const int rank = NW == 8 ? (wu < 4 ? 4 * wgr + wu : 4 * a.n_row_wg + 4 * wgr + wu - 4) : wgr * NW + wu;
    int c = rank;
    if (c < r_nch) fetch(c, std::integral_constant<int, 0>{});
    if constexpr (DEPTH > 1)
        if (c + waves < r_nch) fetch(c + waves, std::integral_constant<int, 1>{});
    // the Q rows go out right after the first chunk; the centroids are staged and the pair table is built
    // while both are on their way, then the Q operands
    // B operands of Q (hi / lo): k-step ks < 4 NB, lane group g, slot i = channel 128(ks>>2) + 32g + 8(ks&3) + i
    float4 qx[2][2];
    if (tid < D) {
        const int bq = tid & 15;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int kg = 2 * (tid >> 4) + e, ks = kg >> 2, gg = kg & 3;
            const int ch = 128 * (ks >> 2) + 32 * gg + 8 * (ks & 3);
            const float * qr = q_row<D>(a, h, bq) + ch;
            qx[e][0] = *(const float4 *) qr;
            qx[e][1] = *(const float4 *) (qr + 4);
        }
    }
    if (tid < 64) s.cent[tid] = tq6_cent(tid);
    // the centroids are in LDS: each wave waits for its own LDS writes, then a bare s_barrier (__syncthreads
    // would also wait for the loads in flight)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll 4
    for (int e = tid; e < 4096; e += 64 * NW) tq6_pair_entry((uint32_t) e, s.cent, s.pt[e]);
    if (tid < D) {
        const int bq = tid & 15;
        const bool live = bq < a.n_rows;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int kg = 2 * (tid >> 4) + e, ks = kg >> 2, gg = kg & 3;
            const float xv[8] = {qx[e][0].x, qx[e][0].y, qx[e][0].z, qx[e][0].w, qx[e][1].x, qx[e][1].y, qx[e][1].z, qx[e][1].w};
            u4 hi, lo;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u2 hl = split2(live ? xv[2 * k] : 0.0f, live ? xv[2 * k + 1] : 0.0f);
                hi[k] = hl.x;
                lo[k] = hl.y;
            }
            *(u4 *) &s.qb[0][ks][gg][bq][0] = hi;
            *(u4 *) &s.qb[1][ks][gg][bq][0] = lo;
        }
    }
    __syncthreads();
    const int c_first = c, c_total = (r_nch - c_first + waves - 1) / waves;
    auto step = [&](auto B) {
        constexpr int bf = decltype(B)::value;
        prio_by_progress((c - c_first) / waves, c_total);
        uint32_t p0, p1;
        chunk(c, p0, p1);
        const bool f16row = f16_chunk(c);
        const int RS = (int) (2 * r_vo);
        const int VO = (int) r_vo;
        wave_sync();     // the previous chunk's readers are done
        if (!f16row) {
            const int words = RS / (int) sizeof(RowWord);
            if (lane < words) {
#pragma unroll
                for (int r = 0; r < A3_CH; ++r) *(RowWord *) (st + r * RS + sizeof(RowWord) * lane) = pfr[bf][r];
            }
        }
        if (c + DEPTH * waves < r_nch) fetch(c + DEPTH * waves, B);
        wave_sync();
        // the arithmetic of the chunk, instantiated for fp16 and for tq6_0 rows (no per-step branches)
        auto math = [&](auto kind) {
            constexpr bool F16 = decltype(kind)::value;
            // scores: A = K values of token n (channels of slot (ks, g, i) as in the Q operand)
            f4 acc[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b] = f4{0, 0, 0, 0};
            // K row of token n: fp16 rows straight from HBM, tq6_0 rows from the staged copy (two pointers,
            // so that each access keeps its own address space)
            const gptr kglob = row_of(p0 + (uint32_t) n < p1 ? p0 + (uint32_t) n : p0);
            const uint8_t * klds = st + n * RS;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 4 * NB; ++ks) {
                const u4 Bh = *(const u4 *) &s.qb[0][ks][g][n][0];
                const u4 Bl = *(const u4 *) &s.qb[1][ks][g][n][0];
                f4 & dst = acc[ks >> 2];
                const int ch = 128 * (ks >> 2) + 32 * g + 8 * (ks & 3);
                if (F16) {
                    const u4 A = *(const __attribute__((address_space(1))) u4 *) (kglob + 2 * ch);
                    dst = mfma32(A, Bh, dst);
                    dst = mfma32(A, Bl, dst);
                } else {
                    u4 Ah, Al;
                    tq6_pairs8(klds + (ks >> 2) * SJKVARN_TQ6_BLOCK_BYTES, 4 * g + (ks & 3), s.pt, Ah, Al);
                    dst = mfma32(Ah, Bh, dst);
                    dst = mfma32(Ah, Bl, dst);
                    dst = mfma32(Al, Bh, dst);
                }
            }
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * g + i;
                float raw;
                if (F16) {
                    raw = NB == 2 ? acc[0][i] + acc[NB - 1][i] : acc[0][i];
                } else {
                    const uint8_t * row = st + r * RS;
                    raw = h2f(*(const uint16_t *) row) * acc[0][i];
                    if (NB == 2) raw += h2f(*(const uint16_t *) (row + SJKVARN_TQ6_BLOCK_BYTES)) * acc[NB - 1][i];
                }
                const uint32_t p = p0 + (uint32_t) r;
                sc[i] = (p < p1 && p < qend) ? raw * r_sc2 : -__builtin_inff();
            }
            const float alpha = softmax_update<4>(sc, m_run, l_run);
            float arow[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * g + i, 64);
            if (__any(arow[0] != 1.0f || arow[1] != 1.0f || arow[2] != 1.0f || arow[3] != 1.0f)) {
#pragma unroll
                for (int j = 0; j < 8 * NB; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) O[j][i] = O[j][i] * arow[i];
            }
            // A operands of PV (k = tokens 4g .. 4g+3): P, times the V block norm for tq6_0 rows
            u2 Ph[NB], Pl[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                    float x[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int r = 4 * g + 2 * pr + e;
                        float nrm = 1.0f;
                        if (!F16) nrm = h2f(*(const uint16_t *) (st + r * RS + VO + b * SJKVARN_TQ6_BLOCK_BYTES));
                        x[e] = sc[2 * pr + e] * nrm;
                    }
                    const u2 hl = split2(x[0], x[1]);
                    Ph[b][pr] = hl.x;
                    Pl[b][pr] = hl.y;
                }
            }
            // B operands of PV: column n of tile j = channel 128(j>>3) + 8n + (j&7), k-slots = tokens 4g .. 4g+3
            // (fp16 V rows straight from HBM: the V half of the K | V entry, rows past p1 repeat row p0)
            gptr vglob[4];
            if (F16) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t p = p0 + (uint32_t) (4 * g + k);
                    vglob[k] = row_of(p < p1 ? p : p0) + 2 * D;
                }
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                u4 vh[4], vl[4];      // per token 4g + k: channels 128b + 8n .. +7 as hi / lo pairs
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (F16) {
                        vh[k] = *(const __attribute__((address_space(1))) u4 *) (vglob[k] + 2 * (128 * b + 8 * n));
                        vl[k] = u4{0, 0, 0, 0};
                    } else {
                        tq6_pairs8(st + (4 * g + k) * RS + VO + b * SJKVARN_TQ6_BLOCK_BYTES, n, s.pt, vh[k], vl[k]);
                    }
                }
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
                    const int wi = jj >> 1;
                    const u2 Bh = u2{__builtin_amdgcn_perm(vh[1][wi], vh[0][wi], sel), __builtin_amdgcn_perm(vh[3][wi], vh[2][wi], sel)};
                    f4 & o = O[8 * b + jj];
                    o = mfma16(Ph[b], Bh, o);
                    o = mfma16(Pl[b], Bh, o);
                    if (!F16) {
                        const u2 Bl = u2{__builtin_amdgcn_perm(vl[1][wi], vl[0][wi], sel), __builtin_amdgcn_perm(vl[3][wi], vl[2][wi], sel)};
                        o = mfma16(Ph[b], Bl, o);
                    }
                }
            }
        };
        if (f16row) math(std::true_type{}); else math(std::false_type{});
    };
    for (;;) {
        if (c >= r_nch) break;
        step(std::integral_constant<int, 0>{});
        c += waves;
        if constexpr (DEPTH > 1) {
            if (c >= r_nch) break;
            step(std::integral_constant<int, 1>{});
            c += waves;
        }
    }
    fin(O, m_run, l_run, [](int j, int nn) { return 128 * (j >> 3) + 8 * nn + (j & 7); });
}

// Up to A3_MAXJ calls (jobs: one layer view, its context and query rows each) share one launch; the
// x workgroups of job j are [wg_base[j], wg_base[j+1]). The jobs sit in the kernel arguments.
constexpr int A3_MAXJ = 8;
struct A3Batch {
    A3Args job[A3_MAXJ];
    int wg_base[A3_MAXJ + 1];
    int slot_base[A3_MAXJ + 1];  // 4/4 kernel: first CU slot of each job
    int n_jobs;
    int n_slots;                 // 4/4 kernel: CU slots of the launch (one workgroup each)
};

static_assert(sizeof(A3Batch) <= 4096, "the job table travels in the kernel arguments");

// unrolled over the table, so that its loads go out together
SJK_DEV int a3_job_of(const A3Batch & b, int x) {
    int j = 0;
#pragma unroll
    for (int k = 1; k < A3_MAXJ; ++k) j += (k < b.n_jobs && x >= b.wg_base[k]) ? 1 : 0;
    return __builtin_amdgcn_readfirstlane(j);
}

// per job: workgroups [0, n_row_wg) stream the sink and the tail, the others sealed records (trellis
// body with BK / BV bits)
// workgroup wg of job a (KV head blockIdx.y)
template <int BK, int BV, int D> __device__ __attribute__((always_inline)) inline void attend3_job(const A3Args & a, int wg) {
    __shared__ A3LdsT<TrLds<BK, BV, D>> s;
    const int h = blockIdx.y;
    if (wg >= a.n_wg) return;                    // a fixed grid (sjk_hip_attend_dyn) may exceed the plan's split
    // the job fields that the first loads depend on, in one round trip (empty asm: the values are needed here)
    asm volatile("" ::"s"(a.n_row_wg), "s"(a.rec_per_wg), "s"(a.n_rec), "s"(a.sink_end), "s"(a.v.S), "s"(a.v.n_head_kv),
                 "s"(a.v.body), "s"(a.v.blocks), "s"(a.n_chunk), "s"(a.sink_chunks), "s"(a.body_end), "s"(a.pend));
    if (wg < a.n_row_wg) {
        a3_rows<1, D>(a, s, h, wg, [&](const f4 * O, float m, float l, auto chan) {
            write_partial<D>(a, s, (float *) s.w.stage, h, wg, O, m, l, 1.0f, chan);
        });
    } else {
        const int r0 = (wg - a.n_row_wg) * a.rec_per_wg;
        const int r1 = r0 + a.rec_per_wg < a.n_rec ? r0 + a.rec_per_wg : a.n_rec;
        a3_trellis<BK, BV, D>(a, s, h, wg, r0, r1);
    }
}

template <int BK, int BV, int D>
__global__ __launch_bounds__(A3_NT) __attribute__((amdgpu_waves_per_eu(2))) void attend3_kernel(const A3Batch b) {
    const int j = a3_job_of(b, blockIdx.x);
    attend3_job<BK, BV, D>(b.job[j], (int) blockIdx.x - b.wg_base[j]);
}


// Log-sum-exp merge of the partials of one (query row, KV head, 64 channels): wave w takes partials
// w, w + 4, ...; every load is issued before any is used (one round trip for up to 64 per wave)
constexpr int A3_CMB_MAX = 256;

// Log-sum-exp merge of the partials of one (query row qi, KV head h, channels 64 qt .. 64 qt + 63): wave w takes
// partials w, w + 4, ...; every load is issued before any is used (one round trip for up to 64 per wave).
// sm / sl / so: LDS for the four waves' results. Partials of 16 rows x (D + 2) floats.
template <int D> SJK_DEV void combine_row(const A3Args & a, int h, int qi, int qt, float * sm, float * sl, float * so) {
    constexpr int PS = A3_Q * (D + 2);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int d = qt * 64 + lane;
    const float * base = a.part + (size_t) h * a.n_wg * PS + qi * (D + 2);
    const int cnt = (a.n_wg - w + 3) / 4;            // partials w + 4 k, k < cnt <= 64
    // the partials' rows in groups of 32, all loads of a group in one round trip (32 registers: with 64 the
    // combine of a batch of many jobs kept fewer workgroups per CU than its grid needs to be resident at once);
    // the first group's loads go out with the (m, l) loads, before the weights are known
    float o[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) o[k] = k < cnt ? base[(size_t) (w + 4 * k) * PS + 2 + d] : 0.0f;
    float mk = -__builtin_inff(), lk = 0.0f;         // lane k holds (m, l) of partial w + 4 k
    if (lane < cnt) {
        const float * p = base + (size_t) (w + 4 * lane) * PS;
        mk = p[0];
        lk = p[1];
    }
    const float M = wave_max(mk);
    const float f = (M == -__builtin_inff() || mk == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mk - M);
    const float L = wave_sum(f * lk);
    float acc = 0.0f;
    for (int k0 = 0; k0 < cnt; k0 += 32) {
        if (k0 > 0) {
#pragma unroll
            for (int k = 0; k < 32; ++k) o[k] = k0 + k < cnt ? base[(size_t) (w + 4 * (k0 + k)) * PS + 2 + d] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k)
            acc = __builtin_fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), k0 + k)), o[k], acc);
    }
    if (lane == 0) { sm[w] = M; sl[w] = L; }
    so[w * 64 + lane] = acc;
    __syncthreads();
    if (w == 0) {
        const float Mt = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
        float Ls = 0.0f, Os = 0.0f;
        if (Mt != -__builtin_inff()) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float fk = sm[k] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sm[k] - Mt);
                Ls = __builtin_fmaf(fk, sl[k], Ls);
                Os = __builtin_fmaf(fk, so[k * 64 + lane], Os);
            }
        }
        const int r = a.row0 + qi, iq = r / a.gq, hq = h * a.gq + r % a.gq;
        a.out[((size_t) iq * a.n_head + hq) * D + d] = Ls == 0.0f ? 0.0f : Os / Ls;
    }
}

// grid (16 rows, KV heads, D / 64 channel blocks x jobs)
template <int D> __global__ __launch_bounds__(A3_NT) void attend3_combine(const A3Batch b) {
    __shared__ float s_M[4], s_L[4], s_O[4][64];
    constexpr int NQ = D / 64;
    static_assert((NQ & (NQ - 1)) == 0, "channel blocks: a power of two");
    const A3Args & a = b.job[blockIdx.z / NQ];
    if ((int) blockIdx.x >= a.n_rows) return;
    combine_row<D>(a, blockIdx.y, blockIdx.x, blockIdx.z & (NQ - 1), s_M, s_L, &s_O[0][0]);
}

// One workgroup of A4_NW wavefronts per CU slot; each slot serves one KV head of one job, as record or as row
// slot.
// CU slot loc of job a. The job must sit in memory the compiler may read again at any time (kernel arguments, or a
// plan written before the launch), not in registers: a spill would be a vector memory operation inside the
// streams' hand-counted vmcnt waits.
template <int D> __device__ __attribute__((always_inline)) inline void attend4_slot(const A3Args & a, int loc) {
    __shared__ A4Lds<D> s;
    asm volatile("" ::"s"(a.slots), "s"(a.rec_slots), "s"(a.rec_a), "s"(a.n_rec), "s"(a.sink_end), "s"(a.v.S),
                 "s"(a.v.n_head_kv), "s"(a.v.body), "s"(a.v.blocks), "s"(a.n_chunk), "s"(a.sink_chunks), "s"(a.body_end),
                 "s"(a.pend));
    const int h = loc / a.slots, ls = loc - h * a.slots;
    if (ls >= a.rec_slots)
        a3_rows<1, D>(a, s, h, ls - a.rec_slots, [&](const f4 * O, float m, float l, auto chan) {
            (void) chan;                         // channel 128(j>>3) + 8n + (j&7) of O tile j, column n
            __syncthreads();                     // the row path's LDS is free once every wave is done
            const int w = (int) threadIdx.x >> 6;
            partial_put<D / 16>(s, (f4 *) &s.r + 1024 * w, O, m, l);
            partial_gather<D>(a, s, (const f4 *) &s.r, 1024, h, ls, [](int d, int & jj, int & nn) {
                jj = 8 * (d >> 7) + (d & 7);
                nn = (d & 127) >> 3;
            });
        });
    else
        a4_records<D>(a, s, h, ls, ls);
}

template <int D>
__global__ __launch_bounds__(A4_NT) __attribute__((amdgpu_waves_per_eu(2))) void attend4_kernel(const A3Batch b) {
    const int slot = (int) blockIdx.x;
    int j = 0;
#pragma unroll
    for (int k = 1; k < A3_MAXJ; ++k) j += (k < b.n_jobs && slot >= b.slot_base[k]) ? 1 : 0;
    j = __builtin_amdgcn_readfirstlane(j);
    attend4_slot<D>(b.job[j], slot - b.slot_base[j]);
}

// ------------------------------------------------------------------------------------------------
// scalar bodies other than 4/4 (attendsc_kernel)
// ------------------------------------------------------------------------------------------------
//
// Scalar records with 2- to 4-bit sides other than 4/4 (4/3, 4/2, 3/4, 3/3, 3/2, 2/4, 2/3, 2/2) at D = 128 or
// 256 (sj_kvarn.h:771-833): a 4-bit side is in the fragment order, a 2- or 3-bit side token-major (the code of
// token t, channel d at bit (t D + d) b of the side's payload). Workgroups of 4 wavefronts, two per CU (the one
// fills the other's barrier waits); a workgroup shares one record in LDS (the next one waits in registers),
// staged with each token-major row padded to an odd number of dwords, so that lanes reading different token rows
// read different banks.
//
// QK (wavefront w: token tiles 2w, 2w + 1, all 16 query rows): the A operand of lane (n, g), k-step ks is the 8
// codes of one token, channels 32 ks + 8g .. +7, decoded straight from the staged record as fp16 subnormals (the
// code c as the half's bits, value c x 2^-24):
//   * token-major: the 8 codes are 8b consecutive bits x; y = x with its upper four codes moved to bit 16
//     (x << (16 - 4b) inserted over x above bit 16), then dword j = (y >> b j) & mask pairs channels (j, j + 4);
//   * fragment order (sj_kvarn.h:807-833): one 16-byte read of the tile's words 4(t & 7) .. +3, dword j =
//     (word j >> 4 nib) & 0x000F000F pairs channels (2j, 2j + 1).
// The Q' operands (Q x Kscale, fp16 hi + lo) are built in the same channel order once per record. P' (P x Vscale
// x 2^k, fp16) goes through LDS in the A-operand order. PV (wavefront w: channel tiles (D / 64) w ..): a 4-bit V
// (fragment order) gives lane (n, g) its B operand (8 tokens of one channel) from one 16-byte read and four
// shift-and-masks, as the K side does; for a token-major V, for each 32-token k-step the wavefront transposes the
// V codes of those tokens and its own channels into its own small table of fp16 subnormals, from which lane (n, g)
// reads its B operand.
// Numerics as the 4/4 kernel: exact codes, Q' hi + lo, P' rounded to fp16 once, fp32 sums, zero points as fp32
// sums.

constexpr int SC_NW = 4;                         // wavefronts per workgroup (two workgroups per CU)
constexpr int SC_NT = 64 * SC_NW;
// halves per token row of a wavefront's V table (its D / 4 channels + 16): the four rows that one transposing
// read takes per 16 lanes fall in different banks (row strides of 40 / 24 dwords), rows 16-byte aligned
template <int D> constexpr int sc_tts() { return D / 4 + 16; }

// the largest staged scalar record (4/3 or 3/4: a 4-bit side, a padded 3-bit side, the scale tables)
template <int D> constexpr int sc_rec_max() { return 64 * D + 128 * (3 * D / 8 + 4) + 6 * D + 768; }

template <int D> struct ScRec {
    alignas(16) uint8_t rec[sc_rec_max<D>()];    // the staged record: K payload | V payload | scale tables
    alignas(16) uint16_t tv[SC_NW][32][sc_tts<D>()];    // per wavefront: 32 tokens x its channels of V codes
    alignas(16) uint16_t qb[2][D / 32][4][A3_Q][8];      // Q' hi / lo in B-operand order [hl][ks][g][query][slot]
    alignas(16) u4 pa[4][64];                    // P' A operands of the four 32-token k-steps
    float corr[SC_NW][A3_Q];
    float wmax[SC_NW][A3_Q];
    float cvp[SC_NW][A3_Q];
    float wl[SC_NW][A3_Q];
};
template <int D> struct ScLds {                  // the record path's tables, or the row path's merge area
    union {
        ScRec<D> s;
        f4 merge[SC_NW][D / 16 * 64];
    };
};
template <int D> using AScLds = A3LdsT<ScLds<D>, SC_NW>;
static_assert(sizeof(AScLds<256>) <= 80 * 1024 && sizeof(AScLds<128>) <= 80 * 1024, "LDS of two workgroups per CU");
static_assert(sc_rec_max<256>() == 31488 && sc_rec_max<128>() == 16384, "largest staged scalar records");

// where the parts of a scalar record sit once staged (token-major rows padded by one dword; an odd dword count)
struct ScStage {
    uint32_t k_row, v_row;                       // bytes of a token-major row (0: the side is in the fragment order)
    uint32_t k_rs, v_rs;                         // staged row stride, bytes
    uint32_t vp, sc;                             // staged offsets of the V payload and of the scale tables
    uint32_t k_upr, v_upr, k_mag, v_mag;         // 16-byte units per row and (65536 / units, rounded up)
};
SJK_DEV ScStage sc_stage(const sj_kvarn_layout & l) {
    ScStage st;
    st.k_row = l.bits_k == 4 ? 0u : (uint32_t) (l.D * l.bits_k / 8);
    st.v_row = l.bits_v == 4 ? 0u : (uint32_t) (l.D * l.bits_v / 8);
    st.k_rs = st.k_row + 4u;
    st.v_rs = st.v_row + 4u;
    const uint32_t ksz = st.k_row ? 128u * st.k_rs : l.v_payload, vsz = st.v_row ? 128u * st.v_rs : l.k_scale - l.v_payload;
    st.vp = (ksz + 15u) & ~15u;
    st.sc = (st.vp + vsz + 15u) & ~15u;
    st.k_upr = st.k_row / 16u;
    st.v_upr = st.v_row / 16u;
    st.k_mag = st.k_upr ? (65536u + st.k_upr - 1u) / st.k_upr : 0u;
    st.v_mag = st.v_upr ? (65536u + st.v_upr - 1u) / st.v_upr : 0u;
    return st;
}

template <int D>
__device__ __attribute__((always_inline)) inline void asc_records(const A3Args & a, AScLds<D> & S, int h, int wgi, int r0, int r1) {
    static_assert(D == 128 || D == 256, "head dimension of the scalar-body kernel");
    constexpr int NKS = D / 32;                  // QK k-steps
    constexpr int NJW = D / 64;                  // PV channel tiles per wavefront
    constexpr int G8W = D / 32;                  // 8-channel groups per wavefront
    constexpr int G8T = D / 128;                 // 8-channel groups per Q' builder thread
    auto & s = S.r.s;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const sjk_hip_view & V = a.v;
    const sj_kvarn_layout & L = V.lay;
    const int H = V.n_head_kv;
    const int bk = L.bits_k, bv = L.bits_v;
    const uint32_t RB = L.bytes;
    const ScStage st = sc_stage(L);
    // the record's bytes, 16 per thread and step (every record is a whole number of 16-byte units, at most
    // 4/3 or 3/4: 112 D + 6 D + 768 bytes); the next record waits in registers while this one is computed
    constexpr int PF = ((112 * D + 6 * D + 768) / 16 + SC_NT - 1) / SC_NT;
    const int nv = (int) (RB / 16u);
    u4 pf[PF];
    auto fetch = [&](int c) {
        const uint32_t gi = (a.sink_end + (uint32_t) c * 128u - V.S) / 128u;
        const uint32_t blk = V.blocks ? V.blocks[gi] : gi;
        const u4 * src = (const u4 *) (V.body + ((size_t) blk * H + h) * RB);
#pragma unroll
        for (int k = 0; k < PF; ++k)
            if (tid + SC_NT * k < nv) pf[k] = src[tid + SC_NT * k];
    };
    if (r0 < r1) fetch(r0);

    // Q' builder role: thread (query bq, 8-channel groups G8T bc .. + G8T - 1, all 8 slots of each)
    const int bq = tid & 15, bc = tid >> 4;
    // slot -> channel within the group: identity for a fragment-order K, (j, j + 4) pairs for a token-major K
    auto kslot_ch = [&](int sl) { return bk == 4 ? sl : (sl >> 1) + 4 * (sl & 1); };
    // layout-only work, done once: each thread's staging destinations
    uint32_t sdst[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        const uint32_t u = (uint32_t) (tid + SC_NT * k), o = 16u * u;
        uint32_t dst;
        if (o < L.v_payload) {
            if (st.k_row) {
                const uint32_t r = (u * st.k_mag) >> 16;
                dst = r * st.k_rs + (o - r * st.k_row);
            } else {
                dst = o;
            }
        } else if (o < L.k_scale) {
            const uint32_t ov = o - L.v_payload;
            if (st.v_row) {
                const uint32_t r = ((ov >> 4) * st.v_mag) >> 16;
                dst = st.vp + r * st.v_rs + (ov - r * st.v_row);
            } else {
                dst = st.vp + ov;
            }
        } else {
            dst = st.sc + (o - L.k_scale);
        }
        sdst[k] = dst;
    }
    float qv[G8T][8];
    {
        const bool live = bq < a.n_rows;
#pragma unroll
        for (int e = 0; e < G8T; ++e) {
            const float * qr = q_row<D>(a, h, bq) + 8 * (G8T * bc + e);
#pragma unroll
            for (int k = 0; k < 8; ++k) qv[e][k] = live ? qr[kslot_ch(k)] : 0.0f;
        }
    }
    const uint32_t qend = q_end(a, n);
    const uint32_t qend_min = q_end(a, 0);       // q_end grows with the row over the live rows
    float m_run = -__builtin_inff(), l_run = 0.0f;   // m shared by the waves, l over the wave's own tokens
    f4 O[NJW];                                   // channel tile NJW w + jj: O[query 4g + i][channel 16 J + n]
#pragma unroll
    for (int j = 0; j < NJW; ++j) O[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t M2 = 0x00010001u;
    uint16_t (*tvw)[sc_tts<D>()] = s.tv[w];      // this wavefront's V table: 32 tokens x its D / 4 channels

    for (int c = r0; c < r1; ++c) {
        prio_by_progress(c - r0, r1 - r0);
        const uint32_t p0 = a.sink_end + (uint32_t) c * 128u;
        __syncthreads();                         // the previous record's readers are done
        // ---- stage the record: token-major rows padded (written as dwords), the rest as it is ----
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            if (tid + SC_NT * k >= nv) continue;
            uint32_t * d = (uint32_t *) (s.rec + sdst[k]);
            d[0] = pf[k].x; d[1] = pf[k].y; d[2] = pf[k].z; d[3] = pf[k].w;
        }
        if (c + 1 < r1) fetch(c + 1);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        const uint8_t * ksc = s.rec + st.sc;                       // Kscale | Kzero | Ktok | Vch | Vscale | Vzero
        const uint32_t o_kze = L.k_zero - L.k_scale, o_ktok = L.k_tok - L.k_scale, o_vch = L.v_ch - L.k_scale,
                       o_vsc = L.v_scale - L.k_scale, o_vze = L.v_zero - L.k_scale;
        // ---- Q' = Q * Kscale (hi / lo) and this thread's part of sum_d Q * Kzero ----
        {
            float corr = 0.0f;
#pragma unroll
            for (int e = 0; e < G8T; ++e) {
                const int gq8 = G8T * bc + e, qks = gq8 >> 2, qg = gq8 & 3;
                // the Kscale / Kzero pairs of slots (2j, 2j + 1): for a token-major K, channels (j, j + 4) of the
                // group, halves j and j + 4 of its 16 bytes; for a fragment-order K, channels (2j, 2j + 1), whose
                // k_ch_idx (sj_kvarn.h:835-841) are j D / 4 + 2 gq8 and that + 1, one dword
                uint32_t ks2[4], kz2[4];
                if (bk == 4) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        ks2[j] = *(const uint32_t *) (ksc + j * (D / 2) + 4 * gq8);
                        kz2[j] = *(const uint32_t *) (ksc + o_kze + j * (D / 2) + 4 * gq8);
                    }
                } else {
                    const u4 W = *(const u4 *) (ksc + 16 * gq8), Z = *(const u4 *) (ksc + o_kze + 16 * gq8);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int lw = j >> 1, hw = 2 + (j >> 1);
                        ks2[j] = j & 1 ? (W[lw] >> 16) | (W[hw] & 0xFFFF0000u) : (W[lw] & 0xFFFFu) | (W[hw] << 16);
                        kz2[j] = j & 1 ? (Z[lw] >> 16) | (Z[hw] & 0xFFFF0000u) : (Z[lw] & 0xFFFFu) | (Z[hw] << 16);
                    }
                }
                u4 hi, lo;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    corr = fma_lo(qv[e][2 * j], kz2[j], corr);
                    corr = fma_hi(qv[e][2 * j + 1], kz2[j], corr);
                    const u2 hl = mul_split(qv[e][2 * j], qv[e][2 * j + 1], ks2[j]);
                    hi[j] = hl.x;
                    lo[j] = hl.y;
                }
                *(u4 *) &s.qb[0][qks][qg][bq][0] = hi;
                *(u4 *) &s.qb[1][qks][qg][bq][0] = lo;
            }
            corr = rows_sum(corr);
            if (g == 0) s.corr[w][bq] = corr;
        }
        __syncthreads();
        // ---- QK: token tiles 2w, 2w + 1 (tokens 32w .. 32w + 31), all k-steps ----
        f4 acc[2], acl[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) { acc[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f}; acl[tt] = acc[tt]; }
        if (bk == 4) {
            const uint32_t sh = 4u * (uint32_t) ((n >> 3) + 2 * (g & 1));
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const u4 Bh = *(const u4 *) &s.qb[0][ks][g][n][0], Bl = *(const u4 *) &s.qb[1][ks][g][n][0];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int tile = (2 * w + tt) * (D / 16) + 2 * ks + (g >> 1);
                    const u4 W = *(const u4 *) (s.rec + 4 * (tile * 32 + 4 * (n & 7)));
                    u4 A;
#pragma unroll
                    for (int j = 0; j < 4; ++j) A[j] = (W[j] >> sh) & 0x000F000Fu;
                    acc[tt] = mfma32(A, Bh, acc[tt]);
                    acl[tt] = mfma32(A, Bl, acl[tt]);
                }
            }
        } else {
            const uint32_t hm = ((1u << (4 * bk)) - 1u) << 16, cm = ((1u << bk) - 1u) * M2;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const u4 Bh = *(const u4 *) &s.qb[0][ks][g][n][0], Bl = *(const u4 *) &s.qb[1][ks][g][n][0];
                const uint32_t bit = (uint32_t) ((32 * ks + 8 * g) * bk);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const uint8_t * row = s.rec + (uint32_t) (32 * w + 16 * tt + n) * st.k_rs;
                    const uint32_t * rw = (const uint32_t *) row + (bit >> 5);
                    const uint32_t x = __builtin_amdgcn_alignbit(rw[1], rw[0], bit & 31u);
                    const uint32_t y = x ^ (hm & ((x << (16 - 4 * bk)) ^ x));   // a bit-field insert
                    u4 A;
#pragma unroll
                    for (int j = 0; j < 4; ++j) A[j] = (y >> (bk * j)) & cm;
                    acc[tt] = mfma32(A, Bh, acc[tt]);
                    acl[tt] = mfma32(A, Bl, acl[tt]);
                }
            }
        }
        // ---- scores (log2 units): S = Ktok * (sum_d Q' c + sum_d Q Kzero) * scale * log2 e; lane (n, g) holds
        // query n, tokens 32w + 16tt + 4g + i ----
        float sc[8];
        {
            float ck = 0.0f;
#pragma unroll
            for (int k = 0; k < SC_NW; ++k) ck += s.corr[k][n];
            const float cs = ck * a.sc2, s24 = a.sc2 * 0x1p24f;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                f4 x;
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = __builtin_fmaf(acc[tt][i] + acl[tt][i], s24, cs);
                const u2 kt = *(const u2 *) (ksc + o_ktok + 2 * (32 * w + 16 * tt + 4 * g));
                sc[4 * tt + 0] = mul_lo(x[0], kt.x);
                sc[4 * tt + 1] = mul_hi(x[1], kt.x);
                sc[4 * tt + 2] = mul_lo(x[2], kt.y);
                sc[4 * tt + 3] = mul_hi(x[3], kt.y);
            }
        }
        if (p0 + 128u > qend_min) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (p0 + (uint32_t) (32 * w + 16 * (e >> 2) + 4 * g + (e & 3)) >= qend) sc[e] = -__builtin_inff();
        }
        // the record's maximum per query, agreed by the four waves
        {
            float mloc = sc[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) mloc = fmaxf(mloc, sc[e]);
            mloc = rows_max(mloc);
            if (g == 0) s.wmax[w][n] = mloc;
        }
        int kx;
        {
            const uint32_t wv = *(const uint32_t *) (ksc + o_vsc + 4 * lane);
            const uint32_t mx = wave_umax(max(wv & 0xFFFFu, wv >> 16));   // non-negative halves order like their bits
            kx = 14 - __builtin_amdgcn_frexp_expf(h2f(mx));
        }
        const float pinv = __builtin_amdgcn_ldexpf(1.0f, -kx);
        __syncthreads();
        float M = s.wmax[0][n];
#pragma unroll
        for (int k = 1; k < SC_NW; ++k) M = fmaxf(M, s.wmax[k][n]);
        const float m_new = fmaxf(m_run, M);
        const bool anyv = m_new != -__builtin_inff();
        const float alpha = anyv ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        // exp2(s - mk) = P * 2^k; a row with no visible token has only -inf scores, and exp2(-inf - 0) = 0
        const float mk = anyv ? m_new - (float) kx : 0.0f;
        float psum = 0.0f, cv = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[4 * tt + i] = __builtin_amdgcn_exp2f(sc[4 * tt + i] - mk);
                psum += sc[4 * tt + i];
            }
            const int t0 = 32 * w + 16 * tt + 4 * g;
            const u2 vs = *(const u2 *) (ksc + o_vsc + 2 * t0);
            const u2 vz = *(const u2 *) (ksc + o_vze + 2 * t0);
            const u2 ah = u2{mul_pk(sc[4 * tt], sc[4 * tt + 1], vs.x), mul_pk(sc[4 * tt + 2], sc[4 * tt + 3], vs.y)};
            cv = fma_lo(sc[4 * tt], vz.x, cv);
            cv = fma_hi(sc[4 * tt + 1], vz.x, cv);
            cv = fma_lo(sc[4 * tt + 2], vz.y, cv);
            cv = fma_hi(sc[4 * tt + 3], vz.y, cv);
            // P' A operand of k-step w: tokens 16 tt + 4g + i of it are k-group 2 tt + g / 2, slots 4 (g & 1) + i
            *(u2 *) ((uint8_t *) &s.pa[w][16 * (2 * tt + (g >> 1)) + n] + 8 * (g & 1)) = ah;
        }
        psum = rows_sum(psum);
        cv = rows_sum(cv);
        if (g == 0) s.cvp[w][n] = cv;
        m_run = m_new;
        l_run = l_run * alpha + psum * pinv;
        float arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int j = 0; j < NJW; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) O[j][i] = O[j][i] * arow[i];
        __syncthreads();
        // ---- PV: channel tiles NJW w + jj, one 32-token k-step at a time; the wavefront first decodes the V codes
        // of the step's tokens x its own channels into its token-major table, 8 channels of a token per 16-byte
        // write (lane: token 32 ks + (lane & 31), channel groups lane / 32 + 2k of its D / 32), then reads its B
        // operands transposed: ds_read_b64_tr_b16 gives lane i of each 16 the element i & 3 of the 8 bytes read by
        // lane 4k + i / 4 as its k-th half, so lane j of lane group g reads row 8g + j / 4 (+ 4), columns
        // 16 jj + 4 (j & 3) .. + 3, and lane n receives tokens 8g .. 8g + 7 of channel 16 jj + n ----
        f4 t[NJW];
        {
            f4 cvr;                              // sum_t P' Vzero of rows 4g + i, in the code scale
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float cr = 0.0f;
#pragma unroll
                for (int k = 0; k < SC_NW; ++k) cr += s.cvp[k][4 * g + i];
                cvr[i] = cr * 0x1p-24f;
            }
#pragma unroll
            for (int jj = 0; jj < NJW; ++jj) t[jj] = cvr;
        }
        const int tl = lane & 31;
        // the 4-bit / token-major choice is made once, outside the k-step loop: inside it, the k-steps' LDS reads
        // are issued together instead of one group per branch
        auto pv_steps = [&](auto v4) {
            constexpr bool V4 = decltype(v4)::value;
            constexpr int NK = G8W / 2;          // 16-byte table writes per lane and k-step
            for (int ks = 0; ks < 4; ++ks) {
                const u4 Ap = s.pa[ks][lane];
                if constexpr (V4) {
                    // fragment order, V side (a = channel, b = token; sj_kvarn.h:807-833): the B operand of lane
                    // (n, g), channel 16 J + n x tokens 8g .. 8g + 7 of the k-step, is words 4 (n & 7) .. +3 of
                    // tile (token tile 2 ks + g / 2, channel tile J), nibble (n >> 3) + 2 (g & 1) for the even token
                    // of each pair and that + 4 for the odd one: dword j = (word j >> 4 nib) & 0x000F000F, no table
                    const uint32_t sh = 4u * (uint32_t) ((n >> 3) + 2 * (g & 1));
#pragma unroll
                    for (int jj = 0; jj < NJW; ++jj) {
                        const int tile = (2 * ks + (g >> 1)) * (D / 16) + NJW * w + jj;
                        const u4 W = *(const u4 *) (s.rec + st.vp + 4 * (tile * 32 + 4 * (n & 7)));
                        u4 Bv;
#pragma unroll
                        for (int j = 0; j < 4; ++j) Bv[j] = (W[j] >> sh) & 0x000F000Fu;
                        t[jj] = mfma32(Ap, Bv, t[jj]);
                    }
                } else {
                    // token-major: the 8 codes of channel group cg of token tk are the bits 8 cg bv .. + 8 bv of its
                    // row; all NK windows are read before any is decoded into the table
                    const int tk = 32 * ks + tl;
                    uint32_t w0[NK], w1[NK];
#pragma unroll
                    for (int k = 0; k < NK; ++k) {
                        const uint32_t bit = (uint32_t) (8 * (G8W * w + (lane >> 5) + 2 * k) * bv);
                        const uint32_t * rw = (const uint32_t *) (s.rec + st.vp + (uint32_t) tk * st.v_rs) + (bit >> 5);
                        w0[k] = rw[0];
                        w1[k] = rw[1];
                    }
#pragma unroll
                    for (int k = 0; k < NK; ++k) {
                        const int lg = (lane >> 5) + 2 * k;   // local channel group
                        const uint32_t bit = (uint32_t) (8 * (G8W * w + lg) * bv);
                        const uint32_t x = __builtin_amdgcn_alignbit(w1[k], w0[k], bit & 31u);
                        u4 pk;                   // channels 8 lg .. +7 as fp16 subnormal pairs (2j, 2j + 1)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            pk[j] = __builtin_amdgcn_ubfe(x, (uint32_t) (2 * j * bv), (uint32_t) bv) |
                                    (__builtin_amdgcn_ubfe(x, (uint32_t) ((2 * j + 1) * bv), (uint32_t) bv) << 16);
                        *(u4 *) &tvw[tl][8 * lg] = pk;
                    }
                    // no wait: one wavefront's LDS instructions execute in order, so its transposing reads below see
                    // the writes above, and the next step's writes come after these reads (the compiler keeps both
                    // orders: they access the same table)
#pragma unroll
                    for (int jj = 0; jj < NJW; ++jj) {
                        typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 hf4;
                        typedef __attribute__((address_space(3))) hf4 * lds_hf4;
                        const int col = 16 * jj + 4 * (n & 3), row = 8 * g + (n >> 2);
                        const u2 b0 = __builtin_bit_cast(u2, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_hf4) &tvw[row][col]));
                        const u2 b1 = __builtin_bit_cast(u2, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_hf4) &tvw[row + 4][col]));
                        t[jj] = mfma32(Ap, u4{b0.x, b0.y, b1.x, b1.y}, t[jj]);
                    }
                }
            }
        };
        if (bv == 4) pv_steps(std::true_type{});
        else pv_steps(std::false_type{});
#pragma unroll
        for (int jj = 0; jj < NJW; ++jj) {
            const int d = 16 * (NJW * w + jj) + n;
            // Vch index v_ch_idx(d) (sj_kvarn.h:843-849) for a fragment-order V, the channel otherwise
            const int vi = bv == 4 ? (d & 7) * (D / 8) + (d >> 4) * 2 + ((d >> 3) & 1) : d;
            const float vch = h2f(*(const uint16_t *) (ksc + o_vch + 2 * vi)) * pinv * 0x1p24f;
#pragma unroll
            for (int i = 0; i < 4; ++i) O[jj][i] = __builtin_fmaf(vch, t[jj][i], O[jj][i]);
        }
    }
    // the partial: m is shared by the waves, l is the sum of their parts, O tiles are disjoint channel slices
    __syncthreads();
    if (g == 0) s.wl[w][n] = l_run;
    __syncthreads();
    float * part = a.part + ((size_t) h * a.n_wg + wgi) * (A3_Q * (D + 2));
#pragma unroll
    for (int jj = 0; jj < NJW; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[(4 * g + i) * (D + 2) + 2 + 16 * (NJW * w + jj) + n] = O[jj][i];
    if (tid < A3_Q) {
        float Ls = 0.0f;
#pragma unroll
        for (int k = 0; k < SC_NW; ++k) Ls += s.wl[k][tid];
        part[tid * (D + 2)] = m_run;
        part[tid * (D + 2) + 1] = Ls;
    }
}

// workgroup wg of job a (KV head blockIdx.y): row workgroups [0, n_row_wg) stream the sink and the tail, the others
// rec_per_wg records each
template <int D> __device__ __attribute__((always_inline)) inline void attendsc_job(const A3Args & a, int wg) {
    __shared__ AScLds<D> s;
    const int h = blockIdx.y;
    if (wg >= a.n_wg) return;                    // a fixed grid (sjk_hip_attend_dyn) may exceed the plan's split
    asm volatile("" ::"s"(a.n_row_wg), "s"(a.rec_per_wg), "s"(a.n_rec), "s"(a.sink_end), "s"(a.v.S), "s"(a.v.n_head_kv),
                 "s"(a.v.body), "s"(a.v.blocks), "s"(a.n_chunk), "s"(a.sink_chunks), "s"(a.body_end), "s"(a.pend));
    if (wg < a.n_row_wg) {
        a3_rows<1, D>(a, s, h, wg, [&](const f4 * O, float m, float l, auto chan) {
            (void) chan;                         // channel 128(j>>3) + 8n + (j&7) of O tile j, column n
            __syncthreads();                     // the row path's LDS is free once every wave is done
            const int w = (int) threadIdx.x >> 6;
            partial_put<D / 16>(s, &s.r.merge[w][0], O, m, l);
            partial_gather<D>(a, s, &s.r.merge[0][0], D / 16 * 64, h, wg, [](int d, int & jj, int & nn) {
                jj = 8 * (d >> 7) + (d & 7);
                nn = (d & 127) >> 3;
            });
        });
    } else {
        const int r0 = (wg - a.n_row_wg) * a.rec_per_wg;
        const int r1 = r0 + a.rec_per_wg < a.n_rec ? r0 + a.rec_per_wg : a.n_rec;
        asc_records<D>(a, s, h, wg, r0, r1);
    }
}

template <int D>
__global__ __launch_bounds__(SC_NT) __attribute__((amdgpu_waves_per_eu(2))) void attendsc_kernel(const A3Batch b) {
    const int j = a3_job_of(b, blockIdx.x);
    attendsc_job<D>(b.job[j], (int) blockIdx.x - b.wg_base[j]);
}


}  // namespace sjk

namespace sjk {

int n_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (!v) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// A launch of the 4/4 kernel writes at most CUs + A3_MAXJ * H partials (one per CU slot; every job takes at least
// one slot per KV head), the trellis and other scalar-body kernels at most 2 CUs + (2 A3_MAXJ + 1) H (about two
// workgroups per CU over the jobs, plus two per job and head for the rounding of its split); 2 CUs + 32 H covers
// both.
int ws_slots(int n_head_kv) { return 2 * n_cus() + 32 * (n_head_kv > 0 ? n_head_kv : 1); }

}  // namespace sjk

using namespace sjk;

static_assert((size_t) A3_PSTRIDE == 16 * (A3_D + 2), "one partial = one workspace slot at D = 256");
static_assert(sizeof(A3Batch) <= WS_PLAN_BYTES, "the 4/4 plan of sjk_hip_attend_dyn fits its workspace area");

extern "C" size_t sjk_hip_workspace_bytes(const sj_kvarn_layout * l, int n_head_kv) {
    if (!l || l->D <= 0 || n_head_kv <= 0) return 0;
    return WS_PLAN_BYTES + ws_stage_bytes(l->D, n_head_kv) +
           (size_t) ws_slots(n_head_kv) * ws_slot_floats(l->D) * sizeof(float);
}

template <int BK, int BV, int D = A3_D> static bool lay_is(const sj_kvarn_layout & l) {
    using RL = RecLay<BK, BV, D>;
    return l.D == D && l.bits_k == BK && l.bits_v == BV && l.bytes == (uint32_t) RL::BYTES && l.k_payload == 0u &&
           l.v_payload == (uint32_t) RL::VPAY && l.k_scale == (uint32_t) RL::KSC && l.k_zero == (uint32_t) RL::KZE &&
           l.k_tok == (uint32_t) RL::KTOK && l.v_ch == (uint32_t) RL::VCH && l.v_scale == (uint32_t) RL::VSC &&
           l.v_zero == (uint32_t) RL::VZE;
}

template <int D> static bool lay_is4(const sj_kvarn_layout & l) {
    using RL = RecLay4<D>;
    return l.D == D && l.bits_k == 4 && l.bits_v == 4 && l.bytes == (uint32_t) RL::BYTES && l.k_payload == 0u &&
           l.v_payload == (uint32_t) RL::VPAY && l.k_scale == (uint32_t) RL::KSC && l.k_zero == (uint32_t) RL::KZE &&
           l.k_tok == (uint32_t) RL::KTOK && l.v_ch == (uint32_t) RL::VCH && l.v_scale == (uint32_t) RL::VSC &&
           l.v_zero == (uint32_t) RL::VZE;
}

// a scalar layout with 2- to 4-bit sides at its sj_kvarn_layout_init offsets (sj_kvarn.h:771-790)
static bool lay_is_scalar(const sj_kvarn_layout & l) {
    if (l.body != SJKVARN_BODY_SCALAR || l.bits_k < 2 || l.bits_k > 4 || l.bits_v < 2 || l.bits_v > 4) return false;
    const uint32_t D = (uint32_t) l.D, G = (uint32_t) l.G;
    const uint32_t vp = D * (uint32_t) l.bits_k / 8u * G, ks = vp + D * (uint32_t) l.bits_v / 8u * G;
    return l.k_payload == 0u && l.v_payload == vp && l.k_scale == ks && l.k_zero == ks + 2u * D &&
           l.k_tok == ks + 4u * D && l.v_ch == ks + 4u * D + 2u * G && l.v_scale == ks + 6u * D + 2u * G &&
           l.v_zero == ks + 6u * D + 4u * G && l.bytes == ks + 6u * D + 6u * G;
}

// kernel instantiation for the body of a layout: 44 (4/4 scalar), 55 (the other scalar bodies), 33 / 32 / 22
// (trellis); all at D = 128 or 256; 0 = none
static int a3_body(const sj_kvarn_layout & l) {
    if (l.G != 128) return 0;
    if (l.body == SJKVARN_BODY_SCALAR) {
        if (lay_is4<256>(l) || lay_is4<128>(l)) return 44;
        return ((l.D == 128 || l.D == 256) && lay_is_scalar(l)) ? 55 : 0;
    }
    if (l.body != SJKVARN_BODY_TRELLIS) return 0;
    if (lay_is<3, 3, 256>(l) || lay_is<3, 3, 128>(l)) return 33;
    if (lay_is<3, 2, 256>(l) || lay_is<3, 2, 128>(l)) return 32;
    if (lay_is<2, 2, 256>(l) || lay_is<2, 2, 128>(l)) return 22;
    return 0;
}

// 1 when these kernels handle the view (every scalar body and the 3/3, 3/2, 2/2 trellis bodies, at D = 128 or 256;
// G = 128; any sink / staging; any number of query rows: they are cut into tiles of 16)
extern "C" int sjk_attend3_supported(const sjk_hip_view * v) {
    return a3_body(v->lay) != 0 &&
           (v->staging == SJKVARN_STAGING_F16 || v->stage_bytes == (v->lay.D / 128) * SJKVARN_TQ6_BLOCK_BYTES);
}

// The plan of one tile: rows row0 .. row0 + n_rows - 1 of every KV head (n_rows <= 16), context regions, chunk and
// record counts; the workgroup split is done later.
__host__ __device__ static void a3_plan(A3Args & a, const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0,
                                        int n_q, int n_head, const float * d_q, float scale, float * d_out, int row0,
                                        int n_rows) {
    a = A3Args{};
    a.v = *v;
    a.N = N; a.qpos0 = qpos0; a.n_q = n_q; a.n_head = n_head;
    a.gq = n_head / v->n_head_kv;
    a.row0 = row0;
    a.n_rows = n_rows;
    a.sc2 = scale * 1.4426950408889634f;
    a.q = d_q; a.out = d_out;
    // the tile's last row sees the most: positions < its query position + 1
    const uint32_t last = qpos0 + (uint32_t) ((row0 + (n_rows > 0 ? n_rows : 1) - 1) / a.gq) + 1u;
    a.pend = N < last ? N : last;
    const uint32_t S = v->S;
    a.sink_end = a.pend < S ? a.pend : S;
    // sealed groups up to the one holding the last visible position; later positions are not read
    uint32_t Bb = B < S ? S : B;
    const uint32_t pend_g = a.pend <= S ? S : S + (a.pend - S + 127u) / 128u * 128u;
    if (Bb > pend_g) Bb = pend_g;
    a.body_end = Bb;
    a.n_rec = (int) ((a.body_end - S) / 128u);
    const uint32_t tail = a.pend > a.body_end ? a.pend - a.body_end : 0u;
    a.sink_chunks = (int) ((a.sink_end + A3_CH - 1) / A3_CH);
    a.n_chunk = a.sink_chunks + (int) ((tail + A3_CH - 1) / A3_CH);
}

// Workgroups of a job for a given work unit (record-equivalents per workgroup): record workgroups take
// ceil(unit) records, sink / tail workgroups about unit / chunk_cost chunks (strided over their waves).
// chunk_cost = the time of one 16-position row chunk in records of the body, from sweeps with the split fitted
// to the slots (a3_fit_unit; a trellis record takes longer than a 4/4 one, so a chunk counts for less).
// Trellis bodies, A3_CHUNK_COST: 0.15 / 0.2 / 0.25 took 64.8 / 57.9 / 57.8 us at configs[3]'s 100K context (3/3t,
// one job, a 5.7K tail), 62.4 / 59.4 / 59.4 us at D = 128 (8 KV heads), and 2.12 / 1.98 / 2.08 ms per configs[4]
// decode round (mean; 8 jobs, 4K-8K tails each; 2.68 ms with 0.4 and no fit).
// Scalar bodies other than 4/4 (attendsc_kernel), A5_CHUNK_COST: 0.2 / 0.25 / 0.3 took 52.8 / 50.1 / 50.0 us
// (3/3s) and 50.4 / 45.7 / 44.9 us (2/4s) at D = 256, 55.7 / 55.0 / 57.9 us and 53.9 / 49.2 / 51.7 us at D = 128.
constexpr double A3_CHUNK_COST = 0.2;
constexpr double A5_CHUNK_COST = 0.3, A5_CHUNK_COST_D128 = 0.25;
__host__ __device__ static double a3_chunk_cost(int body, int D) {
    return body == 55 ? (D == 128 ? A5_CHUNK_COST_D128 : A5_CHUNK_COST) : A3_CHUNK_COST;
}

// trellis: CU slots per KV head, about two workgroups per CU, at most A3_CMB_MAX - 2 per KV head so that a job's
// workgroups (its share plus two for the rounding of its split) stay within what the combine merges
static int a3_slots(int H) {
    const int a3s = (2 * n_cus() + H - 1) / H;
    return a3s < A3_CMB_MAX - 2 ? a3s : A3_CMB_MAX - 2;
}

struct A3Split { int n_row_wg, rec_per_wg, n_rec_wg, n_wg; };
__host__ __device__ static A3Split a3_split_of(int n_rec, int n_chunk, double unit, double chunk_cost) {
    A3Split p;
    p.n_row_wg = n_chunk ? (int) ((chunk_cost * n_chunk + unit - 1e-9) / unit) : 0;
    if (n_chunk && p.n_row_wg < 1) p.n_row_wg = 1;
    p.rec_per_wg = (int) (unit + 1.0 - 1e-9);
    if (p.rec_per_wg < 1) p.rec_per_wg = 1;
    p.n_rec_wg = n_rec ? (n_rec + p.rec_per_wg - 1) / p.rec_per_wg : 0;
    p.n_wg = p.n_row_wg + p.n_rec_wg;
    if (p.n_wg == 0) { p.n_row_wg = 1; p.n_wg = 1; }    // nothing visible: one empty partial per head
    return p;
}

__host__ __device__ static void a3_split(A3Args & a, double unit, double chunk_cost) {
    const A3Split p = a3_split_of(a.n_rec, a.n_chunk, unit, chunk_cost);
    a.n_row_wg = p.n_row_wg;
    a.rec_per_wg = p.rec_per_wg;
    a.n_rec_wg = p.n_rec_wg;
    a.n_wg = p.n_wg;
}

// The work unit of a launch: the proportional one (total work / slots), raised to the next whole number of
// records while the jobs' splits together take more than `slots` workgroups per KV head. Each job rounds its
// record and row workgroups up, so the proportional unit can ask for a few workgroups more than the two per CU
// that are resident at once, and those few then run as a second round after the others (at D = 128, 8 KV heads,
// 100K: 65 workgroups per head for 64 slots took 82 us against 63 us for a split within them).
__host__ __device__ static double a3_fit_unit(const A3Args * jobs, int n_jobs, double unit, double chunk_cost, int slots) {
    int least = 0;                               // one row and one record workgroup per job at the most
    for (int j = 0; j < n_jobs; ++j) {
        const int k = (jobs[j].n_chunk > 0) + (jobs[j].n_rec > 0);
        least += k ? k : 1;
    }
    if (least > slots) return unit;              // no unit fits: keep the proportional one
    for (int it = 0; it < 64; ++it) {
        int sum = 0;
        for (int j = 0; j < n_jobs; ++j) sum += a3_split_of(jobs[j].n_rec, jobs[j].n_chunk, unit, chunk_cost).n_wg;
        if (sum <= slots) break;
        unit = (double) ((long long) unit + 1);
    }
    return unit;
}

// One launch (+ one combine) for jobs that share layout, KV heads and query shape. The work of all
// jobs is cut into about two workgroups per CU (every KV head of every job gets its own workgroups), so
// that the slowest workgroup, which ends the launch, has about the average share.
// 4/4 bodies (attend4_kernel): the launch is cut into CU slots, one per CU (one workgroup of A4_NW
// wavefronts each), shared out over the jobs' KV heads in proportion to their work (a record counts 1, a
// 16-position row chunk A4_CHUNK_COST), and within a KV head into record and row slots. The records of a
// head are cut into equal shares per wavefront (rec_a each, in slot order).
constexpr double A4_CHUNK_COST = 0.8;
// A wavefront streams whole records and whole row chunks, so a slot's time goes in steps: among the numbers of
// records per record wavefront k next to the proportional split's (k - 2 .. k + 2), the split takes the one whose
// larger step count is least, k against A4_CHUNK_UNIT x row chunks per row wavefront, each k with the fewest record
// slots that reach it (the most row slots); the proportional split on a tie. A4_CHUNK_UNIT is the time of a chunk
// in records, from timings at 40K-150K positions (0.5 / 0.65 / 0.8 gave 24.7 / 24.7 / 24.7 us at 40K, 25.9 /
// 25.8 / 26.1 at 50K and the same times at 60K-150K). With the proportional split alone a 40K-50K context gave
// some record wavefronts two records while 16 record slots had none (26.9 / 27.0 us). Seventeen integer
// divisions: the descriptor path runs this in one thread of its plan kernel.
constexpr double A4_CHUNK_UNIT = 0.65;

__host__ __device__ static void a4_split(A3Args & a, int slots) {
    const double rows = A4_CHUNK_COST * a.n_chunk, cost = a.n_rec + rows;
    int ws = 0, rs = 0;
    if (a.n_chunk && a.n_rec) {
        if (slots < 2) slots = 2;
        ws = (int) (rows / cost * slots + 0.5);
        ws = ws < 1 ? 1 : (ws > slots - 1 ? slots - 1 : ws);
        rs = slots - ws;
        // larger step count of a split with r record slots
        auto steps = [&](int r) {
            const int w = slots - r;
            const double k = (double) ((a.n_rec + A4_NW * r - 1) / (A4_NW * r));
            const double c = A4_CHUNK_UNIT * (double) ((a.n_chunk + A4_NW * w - 1) / (A4_NW * w));
            return k > c ? k : c;
        };
        const int k0 = (a.n_rec + A4_NW * rs - 1) / (A4_NW * rs);
        double best = steps(rs);
        int brs = rs;
        for (int k = k0 - 2; k <= k0 + 2; ++k) {
            if (k < 1) continue;
            const int r = (a.n_rec + A4_NW * k - 1) / (A4_NW * k);          // fewest record slots for k
            if (r < 1 || r > slots - 1) continue;
            const double m = steps(r);
            if (m < best - 1e-9) { best = m; brs = r; }
        }
        rs = brs;
        ws = slots - rs;
    } else if (a.n_rec) {
        rs = slots;
    } else {
        ws = slots;                                  // row chunks, or nothing visible (empty partials)
    }
    a.slots = slots;
    a.rec_slots = rs;
    a.rec_a = rs ? (a.n_rec + A4_NW * rs - 1) / (A4_NW * rs) : 0;   // records per wavefront
    a.rec_b = 0;
    a.n_row_wg = ws;
    a.n_rec_wg = rs;
    a.n_wg = slots;
    a.rec_per_wg = 0;
}

// The launch's work shared out over the jobs of bt (slots: 4/4 CU slots per KV head, else workgroups per KV head
// to aim at), each job split into its workgroups, and the job table's bases; the descriptor path runs the same
// code on the device, so that both make the same split. SJK_ERR_UNSUPPORTED when a job would have more partials
// than the combine merges.
__host__ __device__ static int a3_assign(A3Batch & bt, int body, int H, int slots) {
    const bool a4 = body == 44;
    const double cc = a4 ? A4_CHUNK_COST : a3_chunk_cost(body, (int) bt.job[0].v.lay.D);
    double total = 0.0;
    for (int j = 0; j < bt.n_jobs; ++j) total += bt.job[j].n_rec + cc * bt.job[j].n_chunk;
    double unit = total / slots > 1.0 ? total / slots : 1.0;
    if (!a4) unit = a3_fit_unit(bt.job, bt.n_jobs, unit, cc, slots);
    // tiles of one call (jobs on one view: the sequences of a pool share its body but not their block tables and
    // rings): they stream the same records
    bool tiles = bt.n_jobs > 1;
    for (int j = 1; j < bt.n_jobs; ++j) {
        const sjk_hip_view & v = bt.job[j].v, & v0 = bt.job[0].v;
        tiles = tiles && v.body == v0.body && v.blocks == v0.blocks && v.ring == v0.ring && v.sink == v0.sink;
    }
    bt.wg_base[0] = 0;
    bt.slot_base[0] = 0;
    for (int j = 0; j < bt.n_jobs; ++j) {
        A3Args & a = bt.job[j];
        if (a4) {
            const int share = total > 0.0 ? (int) ((a.n_rec + cc * a.n_chunk) / total * slots + 1e-6) : 1;
            a4_split(a, share < 1 ? 1 : share);
        } else {
            a3_split(a, unit, cc);
        }
        if (a.n_wg > A3_CMB_MAX) return SJK_ERR_UNSUPPORTED;
        // the 16-row tiles of a wide call: each tile's workgroups start at a multiple of 8 blocks, so that a tile's
        // workgroup i runs on the XCD of the first tile's workgroup i, which streams the same records at the same
        // time, and reads them from that XCD's L2 (blocks go to the 8 XCDs in turn); the blocks past a tile's split
        // exit at once
        bt.wg_base[j + 1] = bt.wg_base[j] + (tiles ? (a.n_wg + 7) & ~7 : a.n_wg);
        bt.slot_base[j + 1] = bt.slot_base[j] + (a4 ? H * a.slots : 0);
    }
    bt.n_slots = bt.slot_base[bt.n_jobs];
    return 0;
}

static int a3_launch(A3Batch & bt, int body, int H, hipStream_t st) {
    // 4/4: one CU slot per CU; the others: about two workgroups per CU (a3_slots)
    const int slots = body == 44 ? (n_cus() / H > 0 ? n_cus() / H : 1) : a3_slots(H);
    if (a3_assign(bt, body, H, slots)) return SJK_ERR_UNSUPPORTED;
    // the partials of a job go to its view's workspace, after those of the earlier jobs on the same workspace
    void * ws[A3_MAXJ];
    size_t used[A3_MAXJ];
    int n_ws = 0;
    for (int j = 0; j < bt.n_jobs; ++j) {
        A3Args & a = bt.job[j];
        int k = 0;
        while (k < n_ws && ws[k] != a.v.work) ++k;
        if (k == n_ws) { ws[n_ws] = a.v.work; used[n_ws] = 0; ++n_ws; }
        a.part = ws_part(a.v) + used[k] * ws_slot_floats(a.v.lay.D);
        used[k] += (size_t) H * (size_t) a.n_wg;
        if (used[k] > ws_part_slots(a.v)) return SJK_ERR_UNSUPPORTED;   // a workspace below sjk_hip_workspace_bytes
    }
    const dim3 grid((unsigned) bt.wg_base[bt.n_jobs], (unsigned) H);
    const int D = bt.job[0].v.lay.D;
    switch (body) {
    case 44:
        if (D == 128) hipLaunchKernelGGL(attend4_kernel<128>, dim3((unsigned) bt.n_slots), dim3(A4_NT), 0, st, bt);
        else hipLaunchKernelGGL(attend4_kernel<256>, dim3((unsigned) bt.n_slots), dim3(A4_NT), 0, st, bt);
        break;
    case 55:
        if (D == 128) hipLaunchKernelGGL(attendsc_kernel<128>, grid, dim3(SC_NT), 0, st, bt);
        else hipLaunchKernelGGL(attendsc_kernel<256>, grid, dim3(SC_NT), 0, st, bt);
        break;
    case 33:
        if (D == 128) hipLaunchKernelGGL((attend3_kernel<3, 3, 128>), grid, dim3(A3_NT), 0, st, bt);
        else hipLaunchKernelGGL((attend3_kernel<3, 3, 256>), grid, dim3(A3_NT), 0, st, bt);
        break;
    case 32:
        if (D == 128) hipLaunchKernelGGL((attend3_kernel<3, 2, 128>), grid, dim3(A3_NT), 0, st, bt);
        else hipLaunchKernelGGL((attend3_kernel<3, 2, 256>), grid, dim3(A3_NT), 0, st, bt);
        break;
    case 22:
        if (D == 128) hipLaunchKernelGGL((attend3_kernel<2, 2, 128>), grid, dim3(A3_NT), 0, st, bt);
        else hipLaunchKernelGGL((attend3_kernel<2, 2, 256>), grid, dim3(A3_NT), 0, st, bt);
        break;
    default: return SJK_ERR_UNSUPPORTED;
    }
    if (D == 128)
        hipLaunchKernelGGL(attend3_combine<128>, dim3(A3_Q, (unsigned) H, 2u * (unsigned) bt.n_jobs), dim3(A3_NT), 0, st, bt);
    else
        hipLaunchKernelGGL(attend3_combine<256>, dim3(A3_Q, (unsigned) H, 4u * (unsigned) bt.n_jobs), dim3(A3_NT), 0, st, bt);
    return SJK_CHECK_LAUNCH();
}

// n_jobs calls of one layout, KV head count and query shape: the 16-row tiles of every call (the n_q x gq query
// rows of a KV head, in order), A3_MAXJ tiles per launch
extern "C" int sjk_attend3_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale,
                                 void * stream) {
    const int body = a3_body(jobs[0].v.lay), H = jobs[0].v.n_head_kv;
    const int rows = n_q * (n_head / H);
    A3Batch bt = {};
    for (int j = 0; j < n_jobs; ++j) {
        const sjk_hip_attend_job & J = jobs[j];
        for (int r0 = 0; r0 < rows; r0 += A3_Q) {
            a3_plan(bt.job[bt.n_jobs++], &J.v, J.B, J.N, J.qpos0, n_q, n_head, J.d_q, scale, J.d_out, r0,
                    rows - r0 < A3_Q ? rows - r0 : A3_Q);
            const bool last = j + 1 == n_jobs && r0 + A3_Q >= rows;
            if (bt.n_jobs == A3_MAXJ || last) {
                const int rc = a3_launch(bt, body, H, (hipStream_t) stream);
                if (rc) return rc;
                bt = A3Batch{};
            }
        }
    }
    return 0;
}

extern "C" int sjk_attend3(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                           const float * d_q, float scale, float * d_out, void * stream) {
    sjk_hip_attend_job J;
    J.v = *v; J.B = B; J.N = N; J.qpos0 = qpos0; J.d_q = d_q; J.d_out = d_out;
    return sjk_attend3_batch(&J, 1, n_q, n_head, scale, stream);
}

// sjk_hip_attend_dyn: the context bounds come from the descriptor when the kernels run, on a launch shape that
// does not depend on them (4/4: H x slots CU slots; trellis: slots + 2 workgroups per KV head, the most its split
// makes, the ones past the split returning at once). Every workgroup of the call's kernels plans the call itself
// from the same inputs with the host's arithmetic (dyn_plan: a3_plan, then a4_split or a3_split, the same code as
// the host path, so the split and the result are the host path's); no plan kernel and no plan in memory. A
// descriptor the view cannot hold (negative entries, B misaligned or past N, N past n_max, a tail longer than the
// ring) plans a job that reads nothing, and the combine writes NaN rows.
struct DynCall {
    sjk_hip_view v;
    const int32_t * desc;
    uint32_t n_max;
    int n_q, n_head, body;
    int slots;                   // as a3_launch: 4/4 CU slots per KV head, else workgroups per KV head to aim at
    int row0, rows;              // the launch's query rows per KV head [row0, row0 + rows): tiles of 16
    float scale;
    const float * q;
    float * out;
    float * part;
};

// the descriptor: can the view hold it (a refused one plans jobs that read nothing, and the combine writes NaN rows)
SJK_DEV bool dyn_ok(const DynCall & c, uint32_t & B, uint32_t & N, uint32_t & qpos0) {
    const int32_t iB = c.desc[SJK_DESC_B], iN = c.desc[SJK_DESC_N], iQ = c.desc[SJK_DESC_QPOS0];
    B = (uint32_t) iB; N = (uint32_t) iN; qpos0 = (uint32_t) iQ;
    const uint32_t last = qpos0 + (uint32_t) c.n_q, pend = N < last ? N : last, bend = B < c.v.S ? c.v.S : B;
    return iB >= 0 && iN >= 0 && iQ >= 0 && B <= N && N <= c.n_max && (B <= c.v.S || (B - c.v.S) % 128u == 0u) &&
           (pend <= bend || (c.v.ring && c.v.cap >= 16u && pend - bend <= c.v.cap));
}

// tile z of the launch (rows [row0 + 16 z, ..) of the call) as a job of a3_launch, before the split
SJK_DEV bool dyn_tile(const DynCall & c, A3Args & a, int z) {
    uint32_t B, N, qpos0;
    const bool ok = dyn_ok(c, B, N, qpos0);
    const int r0 = A3_Q * z, nr = c.rows - r0 < A3_Q ? c.rows - r0 : A3_Q;
    a3_plan(a, &c.v, B, N, qpos0, c.n_q, c.n_head, c.q, c.scale, c.out, c.row0 + r0, nr);
    if (!ok) { a.n_rec = 0; a.n_chunk = 0; a.sink_chunks = 0; a.n_rows = 0; }
    return ok;
}

// a launch of one tile planned inside each workgroup (the trellis and other scalar bodies): a3_launch's split of
// a single job
__device__ __attribute__((always_inline)) inline bool dyn_plan(const DynCall & c, A3Args & a) {
    const bool ok = dyn_tile(c, a, 0);
    const double cc = a3_chunk_cost(c.body, (int) c.v.lay.D), total = a.n_rec + cc * a.n_chunk;
    a3_split(a, a3_fit_unit(&a, 1, total / c.slots > 1.0 ? total / c.slots : 1.0, cc, c.slots), cc);
    a.part = c.part;
    return ok;
}

// The job table of a launch of several tiles (and of every 4/4 launch), as a3_launch builds it, written by one
// workgroup into the view's workspace: the 4/4 kernel keeps every register busy (planned in registers it spills,
// and a spill's scratch accesses would break its vmcnt counting), and the other kernels would have to plan every
// tile to find their own. The tiles' partials follow each other in the workspace.
__global__ __launch_bounds__(64) void attend_plan_kernel(const DynCall c, A3Batch * plan) {
    __shared__ A3Batch bt;
    if (threadIdx.x == 0) {
        const int nt = (c.rows + A3_Q - 1) / A3_Q;
        bt.n_jobs = nt;
        for (int z = 0; z < nt; ++z) dyn_tile(c, bt.job[z], z);
        a3_assign(bt, c.body, c.v.n_head_kv, c.slots);   // within the combine's reach: the host checked the bound
        size_t used = 0;
        for (int z = 0; z < nt; ++z) {
            bt.job[z].part = c.part + used * ws_slot_floats(c.v.lay.D);
            used += (size_t) c.v.n_head_kv * (size_t) bt.job[z].n_wg;
        }
    }
    __syncthreads();
    static_assert(sizeof(A3Batch) % 4 == 0, "the table as dwords");
    const uint32_t * src = (const uint32_t *) &bt;
    uint32_t * dst = (uint32_t *) plan;
    for (int i = (int) threadIdx.x; i < (int) (sizeof(A3Batch) / 4); i += 64) dst[i] = src[i];
}

template <int D>
__global__ __launch_bounds__(A4_NT) __attribute__((amdgpu_waves_per_eu(2))) void attend4_kernel_dyn(const A3Batch * __restrict__ plan) {
    const int slot = (int) blockIdx.x;
    if (slot >= plan->n_slots) return;           // the grid covers the most slots a table can take
    int j = 0;
#pragma unroll
    for (int k = 1; k < A3_MAXJ; ++k) j += (k < plan->n_jobs && slot >= plan->slot_base[k]) ? 1 : 0;
    j = __builtin_amdgcn_readfirstlane(j);
    attend4_slot<D>(plan->job[j], slot - plan->slot_base[j]);
}

// plan: the launch's job table (several tiles), or null (one tile, planned in the workgroup)
template <int BK, int BV, int D>
__global__ __launch_bounds__(A3_NT) __attribute__((amdgpu_waves_per_eu(2))) void attend3_kernel_dyn(const DynCall c, const A3Batch * __restrict__ plan) {
    if (plan) {
        const int x = (int) blockIdx.x;
        if (x >= plan->wg_base[plan->n_jobs]) return;
        const int j = a3_job_of(*plan, x);
        attend3_job<BK, BV, D>(plan->job[j], x - plan->wg_base[j]);
    } else {
        A3Args a;
        dyn_plan(c, a);
        attend3_job<BK, BV, D>(a, (int) blockIdx.x);
    }
}

template <int D>
__global__ __launch_bounds__(SC_NT) __attribute__((amdgpu_waves_per_eu(2))) void attendsc_kernel_dyn(const DynCall c, const A3Batch * __restrict__ plan) {
    if (plan) {
        const int x = (int) blockIdx.x;
        if (x >= plan->wg_base[plan->n_jobs]) return;
        const int j = a3_job_of(*plan, x);
        attendsc_job<D>(plan->job[j], x - plan->wg_base[j]);
    } else {
        A3Args a;
        dyn_plan(c, a);
        attendsc_job<D>(a, (int) blockIdx.x);
    }
}

// the combine of a descriptor-driven launch (row blockIdx.x of tile blockIdx.z / NQ, KV head blockIdx.y, channels
// 64 (blockIdx.z % NQ) ..; grid z = tiles x D / 64), from the job table, or planned here for a launch of one tile
// without one; a refused descriptor gives NaN rows
template <int D> __global__ __launch_bounds__(A3_NT) void attend3_combine_dyn(const DynCall c, const A3Batch * __restrict__ plan) {
    __shared__ float s_M[4], s_L[4], s_O[4][64];
    constexpr int NQ = D / 64;
    const int z = (int) blockIdx.z / NQ, cb = (int) blockIdx.z % NQ;
    uint32_t B, N, qpos0;
    if (!dyn_ok(c, B, N, qpos0)) {
        const int gq = c.n_head / c.v.n_head_kv, r = A3_Q * z + (int) blockIdx.x, t = (int) threadIdx.x;
        if (r < c.rows && t < 64) {
            const int rr = c.row0 + r, iq = rr / gq, hq = (int) blockIdx.y * gq + rr % gq;
            c.out[((size_t) iq * c.n_head + hq) * D + 64 * cb + t] = __builtin_nanf("");
        }
        return;
    }
    if (plan) {
        const A3Args & a = plan->job[z];
        if ((int) blockIdx.x >= a.n_rows) return;
        combine_row<D>(a, blockIdx.y, blockIdx.x, cb, s_M, s_L, &s_O[0][0]);
    } else {
        A3Args a;
        dyn_plan(c, a);
        if ((int) blockIdx.x >= a.n_rows) return;
        combine_row<D>(a, blockIdx.y, blockIdx.x, cb, s_M, s_L, &s_O[0][0]);
    }
}

extern "C" int sjk_hip_attend_dyn(const sjk_hip_view * v, const int32_t * d_desc, uint32_t n_max, int n_q,
                                  int n_head, const float * d_q, float scale, float * d_out, void * stream) {
    if (!v || !d_desc || !d_q || !d_out || n_q <= 0 || n_head <= 0 || v->n_head_kv <= 0 || n_head % v->n_head_kv)
        return SJKVARN_ERR_ARG;
    const int body = a3_body(v->lay);
    if (!body || !sjk_attend3_supported(v)) {
        set_error("sjk_hip_attend_dyn: the view is not one the attention kernels are built for (a layer's own "
                  "layout: head_dim 128/256, group 128, a scalar body or the 3/3, 3/2, 2/2 trellis body, f16 or tq6_0 "
                  "staging)");
        return SJK_ERR_UNSUPPORTED;
    }
    const int H = v->n_head_kv, cus = n_cus(), D = v->lay.D;
    if (H > cus) return SJK_ERR_UNSUPPORTED;
    // As sjk_hip_attend: the call's query rows per KV head in 16-row tiles, up to A3_MAXJ tiles (jobs) a launch,
    // shared out and split on the device by a3_launch's own arithmetic; a launch and its combine per A3_MAXJ tiles,
    // in stream order. The launch shapes depend on n_q, n_head and the view only: a table's jobs take at most
    // slots + 2 tiles CU slots or workgroups per KV head (4/4: a share below 1 is raised to 1 and a4_split raises
    // it to 2; the others: two for the rounding of each split, and up to 7 more per tile for its alignment to 8
    // blocks); the workgroups past the table's exit at once.
    const int slots = body == 44 ? (cus / H > 0 ? cus / H : 1) : a3_slots(H);
    const int rows = n_q * (n_head / H);
    hipStream_t st = (hipStream_t) stream;
    A3Batch * plan = (A3Batch *) ws_plan(*v);
    for (int r0 = 0; r0 < rows; r0 += A3_Q * A3_MAXJ) {
        const int lrows = rows - r0 < A3_Q * A3_MAXJ ? rows - r0 : A3_Q * A3_MAXJ, nt = (lrows + A3_Q - 1) / A3_Q;
        const int per_head = slots + 2 * nt;                                  // most partials per KV head
        if (nt == 1 && body != 44 && slots + 2 > A3_CMB_MAX) return SJK_ERR_UNSUPPORTED;
        if (ws_part_slots(*v) < (size_t) H * per_head) return SJKVARN_ERR_ARG;
        // blocks per KV head: several tiles of the other bodies start each at a multiple of 8 (a3_assign)
        const int blocks_x = body != 44 && nt > 1 ? per_head + 7 * nt : per_head;
        DynCall c;
        c.v = *v; c.desc = d_desc; c.n_max = n_max; c.n_q = n_q; c.n_head = n_head; c.body = body; c.slots = slots;
        c.row0 = r0; c.rows = lrows;
        c.scale = scale; c.q = d_q; c.out = d_out; c.part = ws_part(*v);
        // a table for 4/4 and for several tiles; one tile of the other bodies is planned in its workgroups
        const bool table = body == 44 || nt > 1;
        if (table) hipLaunchKernelGGL(attend_plan_kernel, dim3(1), dim3(64), 0, st, c, plan);
        const A3Batch * tp = table ? plan : nullptr;
        const dim3 grid((unsigned) blocks_x, (unsigned) H);
        switch (body) {
        case 44: {
            const dim3 g4((unsigned) (H * per_head));
            if (D == 128) hipLaunchKernelGGL(attend4_kernel_dyn<128>, g4, dim3(A4_NT), 0, st, tp);
            else hipLaunchKernelGGL(attend4_kernel_dyn<256>, g4, dim3(A4_NT), 0, st, tp);
            break;
        }
        case 55:
            if (D == 128) hipLaunchKernelGGL(attendsc_kernel_dyn<128>, grid, dim3(SC_NT), 0, st, c, tp);
            else hipLaunchKernelGGL(attendsc_kernel_dyn<256>, grid, dim3(SC_NT), 0, st, c, tp);
            break;
        case 33:
            if (D == 128) hipLaunchKernelGGL((attend3_kernel_dyn<3, 3, 128>), grid, dim3(A3_NT), 0, st, c, tp);
            else hipLaunchKernelGGL((attend3_kernel_dyn<3, 3, 256>), grid, dim3(A3_NT), 0, st, c, tp);
            break;
        case 32:
            if (D == 128) hipLaunchKernelGGL((attend3_kernel_dyn<3, 2, 128>), grid, dim3(A3_NT), 0, st, c, tp);
            else hipLaunchKernelGGL((attend3_kernel_dyn<3, 2, 256>), grid, dim3(A3_NT), 0, st, c, tp);
            break;
        case 22:
            if (D == 128) hipLaunchKernelGGL((attend3_kernel_dyn<2, 2, 128>), grid, dim3(A3_NT), 0, st, c, tp);
            else hipLaunchKernelGGL((attend3_kernel_dyn<2, 2, 256>), grid, dim3(A3_NT), 0, st, c, tp);
            break;
        default: return SJK_ERR_UNSUPPORTED;
        }
        const unsigned nq = (unsigned) (D / 64);
        if (D == 128) hipLaunchKernelGGL(attend3_combine_dyn<128>, dim3(A3_Q, (unsigned) H, nq * (unsigned) nt), dim3(A3_NT), 0, st, c, tp);
        else hipLaunchKernelGGL(attend3_combine_dyn<256>, dim3(A3_Q, (unsigned) H, nq * (unsigned) nt), dim3(A3_NT), 0, st, c, tp);
        if (SJK_CHECK_LAUNCH()) return SJK_ERR_DEVICE;
    }
    return 0;
}
