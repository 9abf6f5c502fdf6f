// sjk_attend.hip - decode attention over a layer's sink, sealed body and staging tail.
//
// Split-K ("flash decoding"): the context [0, N) of one KV head is cut into chunks of whole 128-token
// groups; one workgroup streams one chunk for ALL query rows that map to the KV head (decode width x
// GQA group), so every sealed record is read from HBM once per call instead of once per query row and
// head as in the reference loop (sj_kvarn.h:1535-1564, sj_kvarn_cuda.cuh:102-135). Each workgroup
// keeps an online softmax (m, l, O) per query row and writes it out; a combine kernel merges the
// chunks with the log-sum-exp rule. Results agree with the reference's position-ordered loop within
// fp32 rounding (the reference's own device-vs-host bar is a tolerance, tests/test_cuda.cu:1-2).
#include "sjk_dev.h"

namespace sjk {

constexpr int AT_NT = 256;
constexpr int AT_QROWS = 16;     // query rows per workgroup (decode width x GQA group, per KV head)
constexpr int AT_SUB = 32;       // positions decoded into LDS at a time
constexpr int AT_CHUNK = 512;    // positions per workgroup

struct AttArgs {
    sjk_hip_view v;
    uint32_t B, N, qpos0;
    int n_q, n_head, gq;         // gq = n_head / n_head_kv
    int n_rows;                  // n_q * gq
    int n_chunks;
    float scale;
    const float * q;
    float * out;
    float * part;                // [H][n_chunks][AT_QROWS][D + 2]
};

// K and V value of channel d at position p of KV head h (region resolve, sj_kvarn.h:1516-1533)
SJK_DEV void kv_value(const sjk_hip_view & c, uint32_t B, uint32_t p, int h, int d, float & kv, float & vv) {
    const int D = c.lay.D, H = c.n_head_kv;
    if (p >= c.S && p < B) {
        const uint32_t off = p - c.S, G = (uint32_t) c.lay.G;
        const uint32_t g = off / G;
        const int t = (int) (off % G);
        const uint32_t blk = c.blocks ? c.blocks[g] : g;
        const uint8_t * rec = c.body + ((size_t) blk * H + h) * c.lay.bytes;
        const sj_kvarn_layout & l = c.lay;
        const uint32_t ci = (uint32_t) k_ch_idx(l, d);
        const int bk = l.bits_k, bv = l.bits_v;
        float qk, qv;
        if (l.body == SJKVARN_BODY_TRELLIS) {
            qk = f16_to_f32_fast(codebook(bk, 0)[trellis_window(rec + l.k_payload, bk, d, t)]);
            qv = f16_to_f32_fast(codebook(bv, 1)[trellis_window(rec + l.v_payload, bv, d, t)]);
        } else {
            qk = (float) get_code(rec + l.k_payload, code_bit(l, t, d, 0), bk);
            qv = (float) get_code(rec + l.v_payload, code_bit(l, t, d, 1), bv);
        }
        kv = (qk * get_half(rec, l.k_scale + 2u * ci) + get_half(rec, l.k_zero + 2u * ci)) *
             get_half(rec, l.k_tok + 2u * (uint32_t) t);
        vv = (qv * get_half(rec, l.v_scale + 2u * (uint32_t) t) + get_half(rec, l.v_zero + 2u * (uint32_t) t)) *
             get_half(rec, l.v_ch + 2u * (uint32_t) v_ch_idx(l, d));
        return;
    }
    if (p < c.S && c.sink_type == SJKVARN_SINK_F16) {
        const uint16_t * e = (const uint16_t *) (c.sink + ((size_t) p * H + h) * 4 * D);
        kv = f16_to_f32_fast(e[d]);
        vv = f16_to_f32_fast(e[D + d]);
        return;
    }
    const uint8_t * e = p < c.S ? c.sink + ((size_t) p * H + h) * 2 * c.stage_bytes
                                : c.ring + ((size_t) ((p - c.S) % c.cap) * H + h) * 2 * c.stage_bytes;
    for (int side = 0; side < 2; ++side) {
        const uint8_t * row = e + side * c.stage_bytes;
        float x;
        if (c.staging == SJKVARN_STAGING_F16) {
            x = f16_to_f32_fast(((const uint16_t *) row)[d]);
        } else {
            const uint8_t * blk = row + (size_t) (d >> 7) * SJKVARN_TQ6_BLOCK_BYTES;
            const int j = d & 127;
            const int code = ((blk[2 + (j >> 1)] >> (4 * (j & 1))) & 15) | (((blk[66 + (j >> 2)] >> (2 * (j & 3))) & 3) << 4);
            x = tq6_cent(code) * f16_to_f32_fast((uint16_t) (blk[0] | (blk[1] << 8)));
        }
        if (side == 0) kv = x; else vv = x;
    }
}

template <int D>
__global__ __launch_bounds__(AT_NT) void attend_partial_kernel(AttArgs a) {
    __shared__ float s_q[AT_QROWS][D];
    __shared__ float s_k[AT_SUB][D + 1];
    __shared__ float s_v[AT_SUB][D];
    __shared__ float s_p[AT_QROWS][AT_SUB];
    __shared__ float s_m[AT_QROWS], s_l[AT_QROWS], s_alpha[AT_QROWS];
    const int tid = threadIdx.x, h = blockIdx.y, chunk = blockIdx.x;
    const int H = a.v.n_head_kv;
    for (int e = tid; e < AT_QROWS * D; e += AT_NT) {
        const int qi = e / D, d = e % D;
        float val = 0.0f;
        if (qi < a.n_rows) {
            const int iq = qi / a.gq, hq = h * a.gq + qi % a.gq;
            val = a.q[((size_t) iq * a.n_head + hq) * D + d];
        }
        s_q[qi][d] = val;
    }
    if (tid < AT_QROWS) { s_m[tid] = -__builtin_inff(); s_l[tid] = 0.0f; }
    float o[AT_QROWS];
#pragma unroll
    for (int qi = 0; qi < AT_QROWS; ++qi) o[qi] = 0.0f;
    const uint32_t last = a.qpos0 + (uint32_t) a.n_q;           // no query row sees positions >= last
    const uint32_t pend_all = a.N < last ? a.N : last;
    const uint32_t p_begin = (uint32_t) chunk * AT_CHUNK;
    uint32_t p_end = p_begin + AT_CHUNK;
    if (p_end > pend_all) p_end = pend_all;
    __syncthreads();
    for (uint32_t p0 = p_begin; p0 < p_end; p0 += AT_SUB) {
        for (int e = tid; e < AT_SUB * D; e += AT_NT) {
            const int t = e / D, d = e % D;
            const uint32_t p = p0 + (uint32_t) t;
            float kv = 0.0f, vv = 0.0f;
            if (p < p_end) kv_value(a.v, a.B, p, h, d, kv, vv);
            s_k[t][d] = kv;
            s_v[t][d] = vv;
        }
        __syncthreads();
        for (int e = tid; e < AT_QROWS * AT_SUB; e += AT_NT) {
            const int qi = e / AT_SUB, t = e % AT_SUB;
            const uint32_t p = p0 + (uint32_t) t;
            const uint32_t qpos = a.qpos0 + (uint32_t) (qi / a.gq);
            float s = -__builtin_inff();
            if (qi < a.n_rows && p < p_end && p <= qpos) {
                float acc = 0.0f;
                for (int d = 0; d < D; ++d) acc = acc + s_q[qi][d] * s_k[t][d];
                s = acc * a.scale;
            }
            s_p[qi][t] = s;
        }
        __syncthreads();
        if (tid < AT_QROWS) {
            const int qi = tid;
            float mx = s_m[qi];
            for (int t = 0; t < AT_SUB; ++t) mx = fmaxf(mx, s_p[qi][t]);
            float alpha = 1.0f, sum = 0.0f;
            if (mx != -__builtin_inff()) {
                alpha = __expf(s_m[qi] - mx);
                for (int t = 0; t < AT_SUB; ++t) {
                    const float w = __expf(s_p[qi][t] - mx);
                    s_p[qi][t] = w;
                    sum += w;
                }
            } else {
                for (int t = 0; t < AT_SUB; ++t) s_p[qi][t] = 0.0f;
            }
            s_m[qi] = mx;
            s_l[qi] = s_l[qi] * alpha + sum;
            s_alpha[qi] = alpha;
        }
        __syncthreads();
        for (int d = tid; d < D; d += AT_NT) {
#pragma unroll
            for (int qi = 0; qi < AT_QROWS; ++qi) {
                float acc = o[qi] * s_alpha[qi];
                for (int t = 0; t < AT_SUB; ++t) acc = acc + s_p[qi][t] * s_v[t][d];
                o[qi] = acc;
            }
        }
        __syncthreads();
    }
    float * part = a.part + ((size_t) h * a.n_chunks + chunk) * AT_QROWS * (D + 2);
    for (int d = tid; d < D; d += AT_NT)
#pragma unroll
        for (int qi = 0; qi < AT_QROWS; ++qi) part[qi * (D + 2) + 2 + d] = o[qi];
    if (tid < AT_QROWS) { part[tid * (D + 2)] = s_m[tid]; part[tid * (D + 2) + 1] = s_l[tid]; }
}

template <int D>
__global__ void attend_combine_kernel(AttArgs a) {
    const int h = blockIdx.y, qi = blockIdx.x, d = threadIdx.x;
    if (qi >= a.n_rows) return;
    const float * base = a.part + (size_t) h * a.n_chunks * AT_QROWS * (D + 2) + qi * (D + 2);
    float M = -__builtin_inff();
    for (int c = 0; c < a.n_chunks; ++c) M = fmaxf(M, base[(size_t) c * AT_QROWS * (D + 2)]);
    float L = 0.0f, O = 0.0f;
    if (M != -__builtin_inff()) {
        for (int c = 0; c < a.n_chunks; ++c) {
            const float * pc = base + (size_t) c * AT_QROWS * (D + 2);
            const float m = pc[0];
            if (m == -__builtin_inff()) continue;
            const float w = __expf(m - M);
            L += pc[1] * w;
            O += pc[2 + d] * w;
        }
    }
    const int iq = qi / a.gq, hq = h * a.gq + qi % a.gq;
    a.out[((size_t) iq * a.n_head + hq) * D + d] = L == 0.0f ? 0.0f : O / L;
}

}  // namespace sjk

using namespace sjk;

// growable device workspace for the chunk partials (one per process; calls on one stream are ordered)
static float * g_part = nullptr;
static size_t g_part_bytes = 0;

// the streaming matrix-core kernel (sjk_attend3.hip) for the shapes it is built for
extern "C" int sjk_attend3_supported(const sjk_hip_view * v, int n_rows);
extern "C" int sjk_attend3(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                           const float * d_q, float scale, float * d_out, void * stream);

extern "C" int sjk_attend3_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale,
                                 void * stream);

static bool same_shape(const sjk_hip_view & a, const sjk_hip_view & b) {
    return a.lay.D == b.lay.D && a.lay.G == b.lay.G && a.lay.bits_k == b.lay.bits_k && a.lay.bits_v == b.lay.bits_v &&
           a.lay.body == b.lay.body && a.lay.bytes == b.lay.bytes && a.n_head_kv == b.n_head_kv &&
           a.staging == b.staging && a.stage_bytes == b.stage_bytes;
}

// A view whose visible positions reach past the sealed body needs a ring of at least 16 slots (the kernels
// read a 16-position chunk of the tail with one wrap of the ring at most; layers have >= 128)
static bool tail_ok(const sjk_hip_view & v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q) {
    const uint32_t last = qpos0 + (uint32_t) n_q, pend = N < last ? N : last;
    const uint32_t bend = B < v.S ? v.S : B;
    return pend <= bend || (v.ring && v.cap >= 16u);
}

// Many attention calls in one launch when the matrix-core kernel takes them all (same layout, KV
// heads and staging); otherwise one call per job
extern "C" int sjk_hip_attend_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale,
                                    void * stream) {
    if (n_jobs < 0 || (n_jobs > 0 && !jobs)) return SJKVARN_ERR_ARG;
    if (n_jobs == 0) return 0;
    bool one = true;
    for (int j = 0; j < n_jobs && one; ++j) {
        const sjk_hip_attend_job & J = jobs[j];
        if (!J.d_q || !J.d_out || n_q <= 0 || n_head <= 0 || J.v.n_head_kv <= 0 || n_head % J.v.n_head_kv ||
            !tail_ok(J.v, J.B, J.N, J.qpos0, n_q))
            return SJKVARN_ERR_ARG;
        one = same_shape(J.v, jobs[0].v) && sjk_attend3_supported(&J.v, n_q * (n_head / J.v.n_head_kv));
    }
    if (one) return sjk_attend3_batch(jobs, n_jobs, n_q, n_head, scale, stream);
    for (int j = 0; j < n_jobs; ++j) {
        const sjk_hip_attend_job & J = jobs[j];
        const int rc = sjk_hip_attend(&J.v, J.B, J.N, J.qpos0, n_q, n_head, J.d_q, scale, J.d_out, stream);
        if (rc) return rc;
    }
    return 0;
}

extern "C" int sjk_hip_attend(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                              const float * d_q, float scale, float * d_out, void * stream) {
    if (!v || !d_q || !d_out || n_q <= 0 || n_head <= 0 || v->n_head_kv <= 0 || n_head % v->n_head_kv ||
        !tail_ok(*v, B, N, qpos0, n_q))
        return SJKVARN_ERR_ARG;
    const int gq = n_head / v->n_head_kv;
    if (n_q * gq > AT_QROWS) return SJK_ERR_UNSUPPORTED;
    const int D = v->lay.D;
    if (D != 128 && D != 256) return SJK_ERR_UNSUPPORTED;
    if (sjk_attend3_supported(v, n_q * gq)) return sjk_attend3(v, B, N, qpos0, n_q, n_head, d_q, scale, d_out, stream);
    AttArgs a = {};
    a.v = *v; a.B = B; a.N = N; a.qpos0 = qpos0; a.n_q = n_q; a.n_head = n_head; a.gq = gq; a.n_rows = n_q * gq;
    a.scale = scale; a.q = d_q; a.out = d_out;
    const uint32_t last = qpos0 + (uint32_t) n_q, pend = N < last ? N : last;
    a.n_chunks = (int) ((pend + AT_CHUNK - 1) / AT_CHUNK);
    if (a.n_chunks == 0) a.n_chunks = 1;
    const size_t need = (size_t) v->n_head_kv * a.n_chunks * AT_QROWS * (D + 2) * sizeof(float);
    if (need > g_part_bytes) {
        if (g_part) (void) hipFree(g_part);
        g_part = nullptr; g_part_bytes = 0;
        if (hipMalloc((void **) &g_part, need) != hipSuccess) return SJK_ERR_DEVICE;
        g_part_bytes = need;
    }
    a.part = g_part;
    hipStream_t st = (hipStream_t) stream;
    const dim3 grid((unsigned) a.n_chunks, (unsigned) v->n_head_kv);
    if (D == 256) {
        hipLaunchKernelGGL(attend_partial_kernel<256>, grid, dim3(AT_NT), 0, st, a);
        hipLaunchKernelGGL(attend_combine_kernel<256>, dim3(AT_QROWS, v->n_head_kv), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(attend_partial_kernel<128>, grid, dim3(AT_NT), 0, st, a);
        hipLaunchKernelGGL(attend_combine_kernel<128>, dim3(AT_QROWS, v->n_head_kv), dim3(128), 0, st, a);
    }
    return SJK_CHECK_LAUNCH();
}

namespace sjk {
// K and V rows of positions pos0 .. pos0+n_pos-1 of KV head h (the region resolver on its own)
__global__ void kv_rows_kernel(sjk_hip_view v, uint32_t B, uint32_t pos0, uint32_t n_pos, int h, float * out_k,
                               float * out_v) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int D = v.lay.D;
    if (i >= (size_t) n_pos * D) return;
    const uint32_t p = pos0 + (uint32_t) (i / (size_t) D);
    const int d = (int) (i % (size_t) D);
    float kv, vv;
    kv_value(v, B, p, h, d, kv, vv);
    out_k[i] = kv;
    out_v[i] = vv;
}
}  // namespace sjk

extern "C" int sjk_hip_kv_rows(const sjk_hip_view * v, uint32_t B, uint32_t pos0, uint32_t n_pos, int h, float * d_k,
                               float * d_v, void * stream) {
    if (!v || !d_k || !d_v || h < 0 || h >= v->n_head_kv) return SJKVARN_ERR_ARG;
    const size_t n = (size_t) n_pos * v->lay.D;
    if (!n) return 0;
    hipLaunchKernelGGL(sjk::kv_rows_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, (hipStream_t) stream, *v, B,
                       pos0, n_pos, h, d_k, d_v);
    return SJK_CHECK_LAUNCH();
}
