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

#include <mutex>

namespace sjk {

constexpr int AT_NT = 256;
constexpr int AT_QROWS = 16;     // query rows per workgroup: one tile of the KV head's rows
constexpr int AT_SUB = 32;       // positions decoded into LDS at a time
constexpr int AT_CHUNK = 512;    // positions per workgroup (at least; longer when the workspace is the limit)

// The query rows of a KV head are r = iq * gq + j (query position qpos0 + iq, query head h * gq + j); tile t is
// rows 16 t .. 16 t + 15. A launch takes tiles tile0 .. tile0 + gridDim.z - 1.
struct AttArgs {
    sjk_hip_view v;
    uint32_t B, N, qpos0;
    int n_q, n_head, gq;         // gq = n_head / n_head_kv
    int n_rows;                  // n_q * gq
    int tile0;
    int n_chunks;
    uint32_t chunk;              // positions per chunk (a multiple of AT_SUB)
    float scale;
    const float * q;
    float * out;
    float * part;                // [tile - tile0][H][n_chunks][AT_QROWS][D + 2]
};

// positions visible to the last row of tile t (its rows see [0, min(N, qpos + 1)))
SJK_DEV uint32_t tile_end(const AttArgs & a, int t) {
    const int last = (16 * t + 15 < a.n_rows ? 16 * t + 15 : a.n_rows - 1);
    const uint32_t e = a.qpos0 + (uint32_t) (last / a.gq) + 1u;
    return a.N < e ? a.N : e;
}

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

template <int D> __device__ __attribute__((always_inline)) inline void attend_partial(const AttArgs & a) {
    __shared__ float s_q[AT_QROWS][D];
    __shared__ float s_k[AT_SUB][D + 1];
    __shared__ float s_v[AT_SUB][D];
    __shared__ float s_p[AT_QROWS][AT_SUB];
    __shared__ float s_m[AT_QROWS], s_l[AT_QROWS], s_alpha[AT_QROWS];
    const int tid = threadIdx.x, h = blockIdx.y, chunk = blockIdx.x, tile = a.tile0 + (int) blockIdx.z;
    const int H = a.v.n_head_kv;
    if (chunk >= a.n_chunks) return;              // a fixed grid (sjk_hip_attend_dyn) may exceed the plan's chunks
    const int r0 = 16 * tile;                                    // first row of the tile
    for (int e = tid; e < AT_QROWS * D; e += AT_NT) {
        const int qi = e / D, d = e % D;
        float val = 0.0f;
        if (r0 + qi < a.n_rows) {
            const int r = r0 + qi, iq = r / a.gq, hq = h * a.gq + r % a.gq;
            val = a.q[((size_t) iq * a.n_head + hq) * D + d];
        }
        s_q[qi][d] = val;
    }
    if (tid < AT_QROWS) { s_m[tid] = -__builtin_inff(); s_l[tid] = 0.0f; }
    float o[AT_QROWS];
#pragma unroll
    for (int qi = 0; qi < AT_QROWS; ++qi) o[qi] = 0.0f;
    const uint32_t pend_all = tile_end(a, tile);               // no row of the tile sees positions >= pend_all
    const uint32_t p_begin = (uint32_t) chunk * a.chunk;
    uint32_t p_end = p_begin + a.chunk;
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
            const uint32_t qpos = a.qpos0 + (uint32_t) ((r0 + qi) / a.gq);
            float s = -__builtin_inff();
            if (r0 + qi < a.n_rows && p < p_end && p <= qpos) {
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
    float * part = a.part + (((size_t) blockIdx.z * H + h) * a.n_chunks + chunk) * AT_QROWS * (D + 2);
    for (int d = tid; d < D; d += AT_NT)
#pragma unroll
        for (int qi = 0; qi < AT_QROWS; ++qi) part[qi * (D + 2) + 2 + d] = o[qi];
    if (tid < AT_QROWS) { part[tid * (D + 2)] = s_m[tid]; part[tid * (D + 2) + 1] = s_l[tid]; }
}

template <int D> __global__ __launch_bounds__(AT_NT) void attend_partial_kernel(const AttArgs a) {
    attend_partial<D>(a);
}

template <int D> __device__ __attribute__((always_inline)) inline void attend_combine(const AttArgs & a) {
    const int h = blockIdx.y, qi = blockIdx.x, d = threadIdx.x, tile = a.tile0 + (int) blockIdx.z;
    const int H = a.v.n_head_kv;
    const int r = 16 * tile + qi;
    if (r >= a.n_rows) return;
    const float * base = a.part + ((size_t) blockIdx.z * H + h) * a.n_chunks * AT_QROWS * (D + 2) + qi * (D + 2);
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
    const int iq = r / a.gq, hq = h * a.gq + r % a.gq;
    a.out[((size_t) iq * a.n_head + hq) * D + d] = L == 0.0f ? 0.0f : O / L;
}

template <int D> __global__ void attend_combine_kernel(const AttArgs a) { attend_combine<D>(a); }

// The position chunking of one launch (tiles tile0 .. tile0 + nt - 1): chunks of at least AT_CHUNK positions, as
// many as `slots` partials hold for H x nt (at least one), each a multiple of AT_SUB positions.
__host__ __device__ inline void att_chunks(AttArgs & a, int nt, size_t slots) {
    const int H = a.v.n_head_kv;
    // the launch's last tile sees the most positions
    const int last_row = (a.tile0 + nt) * AT_QROWS - 1 < a.n_rows - 1 ? (a.tile0 + nt) * AT_QROWS - 1 : a.n_rows - 1;
    const uint32_t e = a.qpos0 + (uint32_t) (last_row / a.gq) + 1u, pend = a.N < e ? a.N : e;
    uint32_t n_ch = (pend + AT_CHUNK - 1) / AT_CHUNK;
    const uint32_t max_ch = (uint32_t) (slots / ((size_t) H * nt));
    if (n_ch > max_ch) n_ch = max_ch;
    if (n_ch == 0) n_ch = 1;
    a.chunk = ((pend + n_ch - 1) / n_ch + AT_SUB - 1) / AT_SUB * AT_SUB;
    if (a.chunk == 0) a.chunk = AT_SUB;
    a.n_chunks = (int) n_ch;
}

// sjk_hip_attend_dyn for the layouts of the generic kernel (one tile: up to 16 query rows per KV head): every
// workgroup of the call's two kernels plans the call from the descriptor with the host's arithmetic (att_chunks) on
// a grid sized by n_max, the chunks past the plan's returning at once; a descriptor the view cannot hold plans a
// call that reads nothing (N = 0, no rows) and the combine writes NaN rows.
struct GenDyn {
    sjk_hip_view v;
    const int32_t * desc;
    uint32_t n_max;
    int n_q, n_head;
    float scale;
    const float * q;
    float * out;
    float * part;
    size_t slots;
};

__device__ __attribute__((always_inline)) inline bool gen_plan(const GenDyn & c, AttArgs & a) {
    const int32_t iB = c.desc[SJK_DESC_B], iN = c.desc[SJK_DESC_N], iQ = c.desc[SJK_DESC_QPOS0];
    const uint32_t B = (uint32_t) iB, N = (uint32_t) iN, qpos0 = (uint32_t) iQ;
    const uint32_t last = qpos0 + (uint32_t) c.n_q, pend = N < last ? N : last, bend = B < c.v.S ? c.v.S : B;
    const bool ok = iB >= 0 && iN >= 0 && iQ >= 0 && B <= N && N <= c.n_max &&
                    (B <= c.v.S || (B - c.v.S) % (uint32_t) c.v.lay.G == 0u) &&
                    (pend <= bend || (c.v.ring && c.v.cap >= 16u && pend - bend <= c.v.cap));
    a = AttArgs{};
    a.v = c.v; a.B = ok ? B : 0u; a.N = ok ? N : 0u; a.qpos0 = ok ? qpos0 : 0u;
    a.n_q = c.n_q; a.n_head = c.n_head; a.gq = c.n_head / c.v.n_head_kv;
    a.n_rows = ok ? c.n_q * a.gq : 0;
    a.scale = c.scale; a.q = c.q; a.out = c.out; a.part = c.part;
    a.tile0 = 0;
    att_chunks(a, 1, c.slots);
    return ok;
}

template <int D> __global__ __launch_bounds__(AT_NT) void attend_partial_kernel_dyn(const GenDyn c) {
    AttArgs a;
    gen_plan(c, a);
    attend_partial<D>(a);
}

template <int D> __global__ void attend_combine_kernel_dyn(const GenDyn c) {
    AttArgs a;
    if (!gen_plan(c, a)) {
        const int gq = c.n_head / c.v.n_head_kv, r = (int) blockIdx.x;
        if (r < c.n_q * gq) {
            const int iq = r / gq, hq = (int) blockIdx.y * gq + r % gq;
            c.out[((size_t) iq * c.n_head + hq) * D + threadIdx.x] = __builtin_nanf("");
        }
        return;
    }
    attend_combine<D>(a);
}

}  // namespace sjk

using namespace sjk;

// the streaming matrix-core kernels (sjk_attend3.hip) for the layouts they are built for
extern "C" int sjk_attend3_supported(const sjk_hip_view * v);
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

static bool args_ok(const sjk_hip_view & v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head, const float * q,
                    const float * out) {
    return q && out && n_q > 0 && n_head > 0 && v.n_head_kv > 0 && n_head % v.n_head_kv == 0 && v.work &&
           tail_ok(v, B, N, qpos0, n_q);
}

// Many attention calls in one launch when the matrix-core kernel takes them all (same layout, KV
// heads and staging); otherwise one call per job
extern "C" int sjk_hip_attend_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale,
                                    void * stream) {
    if (n_jobs < 0 || (n_jobs > 0 && !jobs)) return SJKVARN_ERR_ARG;
    if (n_jobs == 0) return 0;
    bool one = true;
    for (int j = 0; j < n_jobs; ++j) {
        const sjk_hip_attend_job & J = jobs[j];
        if (!args_ok(J.v, J.B, J.N, J.qpos0, n_q, n_head, J.d_q, J.d_out)) return SJKVARN_ERR_ARG;
        one = one && same_shape(J.v, jobs[0].v) && sjk_attend3_supported(&J.v);
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
    if (!v || !args_ok(*v, B, N, qpos0, n_q, n_head, d_q, d_out)) return SJKVARN_ERR_ARG;
    const int D = v->lay.D, H = v->n_head_kv;
    if (D != 128 && D != 256) return SJK_ERR_UNSUPPORTED;
    if (sjk_attend3_supported(v)) return sjk_attend3(v, B, N, qpos0, n_q, n_head, d_q, scale, d_out, stream);
    // the generic kernel: tiles of 16 rows, up to 8 tiles per launch, as many position chunks (of at least
    // AT_CHUNK positions) as the workspace holds partials for
    AttArgs a = {};
    a.v = *v; a.B = B; a.N = N; a.qpos0 = qpos0; a.n_q = n_q; a.n_head = n_head; a.gq = n_head / H;
    a.n_rows = n_q * a.gq;
    a.scale = scale; a.q = d_q; a.out = d_out; a.part = ws_part(*v);
    const int n_tiles = (a.n_rows + AT_QROWS - 1) / AT_QROWS;
    const size_t slots = ws_part_slots(*v);
    int tpl = n_tiles < 8 ? n_tiles : 8;
    if ((size_t) (H * tpl) > slots) tpl = (int) (slots / (size_t) H);
    if (tpl < 1) return SJKVARN_ERR_ARG;                        // a workspace below sjk_hip_workspace_bytes
    hipStream_t st = (hipStream_t) stream;
    for (a.tile0 = 0; a.tile0 < n_tiles; a.tile0 += tpl) {
        const int nt = n_tiles - a.tile0 < tpl ? n_tiles - a.tile0 : tpl;
        att_chunks(a, nt, slots);
        const dim3 grid((unsigned) a.n_chunks, (unsigned) H, (unsigned) nt);
        if (D == 256) {
            hipLaunchKernelGGL(attend_partial_kernel<256>, grid, dim3(AT_NT), 0, st, a);
            hipLaunchKernelGGL(attend_combine_kernel<256>, dim3(AT_QROWS, H, nt), dim3(256), 0, st, a);
        } else {
            hipLaunchKernelGGL(attend_partial_kernel<128>, grid, dim3(AT_NT), 0, st, a);
            hipLaunchKernelGGL(attend_combine_kernel<128>, dim3(AT_QROWS, H, nt), dim3(128), 0, st, a);
        }
        const int rc = SJK_CHECK_LAUNCH();
        if (rc) return rc;
    }
    return 0;
}

// sjk_hip_attend_dyn for views the matrix-core kernels do not take (D = 128, other bodies, bit widths): a fixed grid
// of as many chunks as n_max positions give (capped by the workspace), the ones past the plan's chunking returning
extern "C" int sjk_attend_dyn_generic(const sjk_hip_view * v, const int32_t * d_desc, uint32_t n_max, int n_q,
                                      int n_head, const float * d_q, float scale, float * d_out, void * stream) {
    const int D = v->lay.D, H = v->n_head_kv;
    if (D != 128 && D != 256) return SJK_ERR_UNSUPPORTED;
    if (n_q * (n_head / H) > AT_QROWS) return SJK_ERR_UNSUPPORTED;
    if (!v->work) return SJKVARN_ERR_ARG;
    const size_t slots = ws_part_slots(*v);
    if (slots < (size_t) H) return SJKVARN_ERR_ARG;              // a workspace below sjk_hip_workspace_bytes
    uint32_t n_ch = (n_max + AT_CHUNK - 1) / AT_CHUNK;
    if (n_ch > slots / (size_t) H) n_ch = (uint32_t) (slots / (size_t) H);
    if (n_ch == 0) n_ch = 1;
    GenDyn c;
    c.v = *v; c.desc = d_desc; c.n_max = n_max; c.n_q = n_q; c.n_head = n_head; c.scale = scale; c.q = d_q;
    c.out = d_out; c.part = ws_part(*v); c.slots = slots;
    hipStream_t st = (hipStream_t) stream;
    const dim3 grid(n_ch, (unsigned) H, 1u);
    if (D == 256) {
        hipLaunchKernelGGL(attend_partial_kernel_dyn<256>, grid, dim3(AT_NT), 0, st, c);
        hipLaunchKernelGGL(attend_combine_kernel_dyn<256>, dim3(AT_QROWS, H, 1), dim3(256), 0, st, c);
    } else {
        hipLaunchKernelGGL(attend_partial_kernel_dyn<128>, grid, dim3(AT_NT), 0, st, c);
        hipLaunchKernelGGL(attend_combine_kernel_dyn<128>, dim3(AT_QROWS, H, 1), dim3(128), 0, st, c);
    }
    return SJK_CHECK_LAUNCH();
}

// ---- sjk_hip_attend_noalloc: sjk_hip_attend with its workspace in a static device array ----
// Callers that cannot allocate device memory (code under stream capture, serving loops that forbid hipMalloc)
// pass views without a workspace; the partial results then go to `scratch`, one array per device, held until
// the process ends. In host code the array's name is only a stand-in: its device address comes from
// hipGetSymbolAddress, taken once per device with that device current and kept in g_scratch[dev].
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t) 16 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void * g_scratch[64];

static void * scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void * p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        g_scratch[dev] = p;
    }
    return g_scratch[dev];
}

extern "C" int sjk_hip_attend_noalloc(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q,
                                      int n_head, const float * d_q, float scale, float * d_out, void * stream) {
    if (!v || v->n_head_kv <= 0) return SJKVARN_ERR_ARG;
    const size_t need = sjk_hip_workspace_bytes(&v->lay, v->n_head_kv);
    if (need == 0 || need > NOALLOC_SCRATCH_BYTES) {
        set_error("sjk_hip_attend_noalloc: the view's workspace size exceeds the 16 MiB static scratch "
                  "(head_dim x KV heads too large)");
        return SJKVARN_ERR_CAPACITY;
    }
    void * p = scratch_ptr();
    if (!p) return SJK_ERR_DEVICE;
    sjk_hip_view w = *v;
    w.work = p;
    w.work_bytes = NOALLOC_SCRATCH_BYTES;
    return sjk_hip_attend(&w, B, N, qpos0, n_q, n_head, d_q, scale, d_out, stream);
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
