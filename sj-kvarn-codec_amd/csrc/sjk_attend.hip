// sjk_attend.hip - the decode-attention entry points (sjk_hip_attend, _batch, _noalloc) and the region resolver
// on its own (sjk_hip_kv_rows).
//
// The attention itself runs on the streaming matrix-core kernels of sjk_attend3.hip, which take every layout a
// layer can have (D = 128 or 256, G = 128, every scalar body and the 3/3, 3/2, 2/2 trellis bodies, f16 or tq6_0
// staging). A hand-built view outside those (another G, D or record layout) is refused with SJK_ERR_UNSUPPORTED
// and a message, before any GPU call. Results agree with the reference's position-ordered loop
// (sj_kvarn.h:1535-1564, sj_kvarn_cuda.cuh:102-135) within fp32 rounding (the reference's own device-vs-host bar
// is a tolerance, tests/test_cuda.cu:1-2).
#include "sjk_dev.h"

#include <mutex>
#include <stdio.h>

namespace sjk {

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
        kv = dequant_x(qk, get_half(rec, l.k_scale + 2u * ci), get_half(rec, l.k_zero + 2u * ci),
                       get_half(rec, l.k_tok + 2u * (uint32_t) t));
        vv = dequant_x(qv, get_half(rec, l.v_scale + 2u * (uint32_t) t), get_half(rec, l.v_zero + 2u * (uint32_t) t),
                       get_half(rec, l.v_ch + 2u * (uint32_t) v_ch_idx(l, d)));
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
            x = xmul(tq6_cent(code), f16_to_f32((uint16_t) (blk[0] | (blk[1] << 8))));
        }
        if (side == 0) kv = x; else vv = x;
    }
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

static int unsupported(const char * who) {
    char msg[256];
    snprintf(msg, sizeof msg, "%s: the view is not one the attention kernels are built for (a layer's own layout: "
             "head_dim 128/256, group 128, a scalar body or the 3/3, 3/2, 2/2 trellis body, f16 or tq6_0 staging)", who);
    set_error(msg);
    return SJK_ERR_UNSUPPORTED;
}

// Many attention calls in one launch when they share the layout, KV heads and staging; otherwise one call per job.
// Every job is checked before anything is launched.
extern "C" int sjk_hip_attend_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale,
                                    void * stream) {
    if (n_jobs < 0 || (n_jobs > 0 && !jobs)) return SJKVARN_ERR_ARG;
    if (n_jobs == 0) return 0;
    bool one = true;
    for (int j = 0; j < n_jobs; ++j) {
        const sjk_hip_attend_job & J = jobs[j];
        if (!args_ok(J.v, J.B, J.N, J.qpos0, n_q, n_head, J.d_q, J.d_out)) return SJKVARN_ERR_ARG;
        if (!sjk_attend3_supported(&J.v)) return unsupported("sjk_hip_attend_batch");
        one = one && same_shape(J.v, jobs[0].v);
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
    if (!sjk_attend3_supported(v)) return unsupported("sjk_hip_attend");
    return sjk_attend3(v, B, N, qpos0, n_q, n_head, d_q, scale, d_out, stream);
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
    if (!sjk_attend3_supported(v)) return unsupported("sjk_hip_attend_noalloc");
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
