// sjk_rows.hip - row kernels: Hadamard rotation, tq6_0 / fp16 staging (the append path), unstaging,
// and record decode.
//
// Row kernels run one wavefront per row of D = 64*V values; lane l holds values V*l .. V*l+V-1.
//   * Hadamard (sj_kvarn.h:735-752): stages h < V inside a lane, stages h >= V between lanes l and
//     l ^ (h/V); the lower partner keeps a+b, the upper a-b (a = lower value), then one multiply by
//     1/sqrt(D). Same stage order and operations as the reference, so bit-identical.
//   * tq6_0 (sj_kvarn.h:1221-1247): the two per-block sums (x^2, then centroid^2) must be sequential
//     fp32 sums over the 128 values in index order. The squares are formed in parallel, written to
//     LDS, and every lane of the block walks them in order with broadcast reads, so each lane ends
//     with the block's exact sum. The level search, packing and stores are parallel over lanes.
#include "sjk_dev.h"

namespace sjk {

constexpr int ROW_WAVES = 4;                 // wavefronts (rows) per workgroup
enum { OUT_F32 = 0, OUT_F16 = 1, OUT_TQ6 = 2 };

struct RowJob {
    int kind;            // 0: plain rows (stage/rotate), 1: layer store
    int D;
    int n_rows;
    int rotate;
    float rot_scale;     // RN(1/sqrt(D)), computed on the host (IEEE, same as sqrtf then /)
    // kind 0
    const float * x;
    uint8_t * dst;
    size_t dst_row_bytes;
    int out_mode;
    // kind 1 (sj_kvarn_layer_store, sj_kvarn.h:1475-1492)
    const float * k;
    const float * v;
    uint8_t * sink;
    uint8_t * ring;
    uint32_t pos0, S, cap;
    int H, sink_type, staging;
    size_t stage_bytes;
    const int32_t * pos_desc;   // sjk_hip_layer_store_dyn: pos0 = pos_desc[SJK_DESC_QPOS0], read when the kernel runs
};

SJK_DEV void job_row(const RowJob & j, int r, const float *& src, uint8_t *& dst, int & mode) {
    if (j.kind == 0) {
        src = j.x + (size_t) r * j.D;
        dst = j.dst + (size_t) r * j.dst_row_bytes;
        mode = j.out_mode;
        return;
    }
    const int side = r & 1, hh = (r >> 1) % j.H, ip = (r >> 1) / j.H;
    const uint32_t pos = (j.pos_desc ? (uint32_t) j.pos_desc[SJK_DESC_QPOS0] : j.pos0) + (uint32_t) ip;
    src = (side ? j.v : j.k) + ((size_t) ip * j.H + hh) * j.D;
    if (pos < j.S && j.sink_type == SJKVARN_SINK_F16) {
        dst = j.sink + ((size_t) pos * j.H + hh) * 4 * j.D + (size_t) side * 2 * j.D;
        mode = OUT_F16;
        return;
    }
    uint8_t * e = pos < j.S ? j.sink + ((size_t) pos * j.H + hh) * 2 * j.stage_bytes
                            : j.ring + ((size_t) ((pos - j.S) % j.cap) * j.H + hh) * 2 * j.stage_bytes;
    dst = e + (size_t) side * j.stage_bytes;
    mode = j.staging == SJKVARN_STAGING_F16 ? OUT_F16 : OUT_TQ6;
}

// up to ROW_MAXJ jobs per launch: rows [row_base[k], row_base[k+1]) of the grid belong to job k
constexpr int ROW_MAXJ = 16;
struct RowBatch {
    RowJob job[ROW_MAXJ];
    int row_base[ROW_MAXJ + 1];
    int n_jobs;
};

static_assert(sizeof(RowBatch) <= 4096, "the job table travels in the kernel arguments");

// Hadamard of one row held V values per lane (sj_kvarn.h:735-752): stages h < V inside the lane, stages h >= V
// between lanes l and l ^ (h / V) (the lower partner keeps a + b, the upper a - b, a = the lower value), then one
// multiply by 1/sqrt(D). XN: the host's NaN rule (a row holding an infinity or a NaN).
template <int V, bool XN>
SJK_DEV void hadamard_row(float (&x)[V], int lane, float scale) {
#pragma unroll
    for (int h = 1; h < V; h *= 2)
#pragma unroll
        for (int m = 0; m < V; ++m)
            if (!(m & h)) {
                const float a = x[m], b = x[m + h];
                x[m] = XN ? xadd(a, b) : a + b;
                x[m + h] = XN ? xsub(a, b) : a - b;
            }
#pragma unroll
    for (int lm = 1; lm < 64; lm *= 2) {
        const bool upper = (lane & lm) != 0;
#pragma unroll
        for (int m = 0; m < V; ++m) {
            const float o = __shfl_xor(x[m], lm, 64);
            x[m] = upper ? (XN ? xsub(o, x[m]) : o - x[m]) : (XN ? xadd(x[m], o) : x[m] + o);
        }
    }
#pragma unroll
    for (int m = 0; m < V; ++m) x[m] = XN ? xmul(x[m], scale) : x[m] * scale;
}

template <int V>
__global__ __launch_bounds__(64 * ROW_WAVES) void rows_kernel(const RowBatch bt) {
    constexpr int D = 64 * V;
    __shared__ float s_sq[ROW_WAVES][D];
    __shared__ float s_mid[64], s_cent[64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x < 64) {
        s_mid[threadIdx.x] = threadIdx.x < 63 ? tq6_mid(threadIdx.x) : __builtin_inff();
        s_cent[threadIdx.x] = tq6_cent(threadIdx.x);
    }
    const int rg = blockIdx.x * ROW_WAVES + wave;             // wave-uniform
    int ji = 0;
    for (int k = 1; k < bt.n_jobs; ++k) ji += rg >= bt.row_base[k] ? 1 : 0;
    ji = __builtin_amdgcn_readfirstlane(ji);
    const RowJob & j = bt.job[ji];
    const int r = rg - bt.row_base[ji];
    const bool live = rg < bt.row_base[bt.n_jobs] && !(j.pos_desc && j.pos_desc[SJK_DESC_QPOS0] < 0);
    const float * src = nullptr;
    uint8_t * dst = nullptr;
    int mode = OUT_F32;
    float x[V];
#pragma unroll
    for (int m = 0; m < V; ++m) x[m] = 0.0f;
    if (live) {
        job_row(j, r, src, dst, mode);
#pragma unroll
        for (int m = 0; m < V; ++m) x[m] = src[V * lane + m];
    }
    // a row holding an infinity or a NaN takes the rotation and the tq6_0 sums with the host's NaN rule (wave-uniform)
    bool nf = false;
#pragma unroll
    for (int m = 0; m < V; ++m) nf |= (f_bits(x[m]) & 0x7F800000u) == 0x7F800000u;
    const bool xn = __any(nf);
    if (live && j.rotate) {
        if (xn) hadamard_row<V, true>(x, lane, j.rot_scale);
        else hadamard_row<V, false>(x, lane, j.rot_scale);
    }
    __syncthreads();
    if (live && mode == OUT_F32) {
        float * o = (float *) dst;
#pragma unroll
        for (int m = 0; m < V; ++m) o[V * lane + m] = x[m];
    }
    if (live && mode == OUT_F16) {
        uint16_t * o = (uint16_t *) dst;
#pragma unroll
        for (int m = 0; m < V; ++m) o[V * lane + m] = f32_to_f16(x[m]);
    }
    // tq6_0: every wave takes part in the barriers; only tq6 rows use the results
    constexpr int LPB = 128 / V;           // lanes per 128-value block
    const int b = lane / LPB;              // block of this lane
    float * sq = s_sq[wave];
#pragma unroll
    for (int m = 0; m < V; ++m) sq[V * lane + m] = xn ? xmul(x[m], x[m]) : x[m] * x[m];
    __syncthreads();
    float nsq = 0.0f;
    {
        const float4 * p = (const float4 *) (sq + 128 * b);
        if (xn) {
            for (int i = 0; i < 32; ++i) {
                const float4 q = p[i];
                nsq = xadd(nsq, q.x); nsq = xadd(nsq, q.y); nsq = xadd(nsq, q.z); nsq = xadd(nsq, q.w);
            }
        } else {
#pragma unroll 8
            for (int i = 0; i < 32; ++i) {
                const float4 q = p[i];
                nsq = nsq + q.x; nsq = nsq + q.y; nsq = nsq + q.z; nsq = nsq + q.w;
            }
        }
    }
    const float norm = nsq != nsq ? nan_of(nsq) : __builtin_sqrtf(nsq);
    const bool big = norm > 1e-10f;
    const float inv = big ? 1.0f / norm : 0.0f;
    int code[V];
#pragma unroll
    for (int m = 0; m < V; ++m) code[m] = tq6_level(big ? x[m] * inv : 0.0f, s_mid);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < V; ++m) { const float c = s_cent[code[m]]; sq[V * lane + m] = c * c; }
    __syncthreads();
    float rsq = 0.0f;
    {
        const float4 * p = (const float4 *) (sq + 128 * b);
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            const float4 q = p[i];
            rsq = rsq + q.x; rsq = rsq + q.y; rsq = rsq + q.z; rsq = rsq + q.w;
        }
    }
    const float rn = __builtin_sqrtf(rsq);
    if (!(live && mode == OUT_TQ6)) return;
    uint8_t * blk = dst + (size_t) b * SJKVARN_TQ6_BLOCK_BYTES;
    const int i0 = V * (lane % LPB);       // index of this lane's first value inside its block
    if (lane % LPB == 0) *(uint16_t *) blk = f32_to_f16(rn > 1e-10f ? xdiv(norm, rn) : norm);
    // low nibbles: qs[i/2] bit 4*(i%2); high pairs: qh[i/4] bit 2*(i%4)
    uint32_t qs = 0, qh = 0;
#pragma unroll
    for (int m = 0; m < V; ++m) {
        qs |= (uint32_t) (code[m] & 15) << (4 * m);
        qh |= (uint32_t) ((code[m] >> 4) & 3) << (2 * m);
    }
    if (V == 2) {
        // two lanes share one qh byte
        const uint32_t other = (uint32_t) __shfl_xor((int) qh, 1, 64);
        blk[2 + i0 / 2] = (uint8_t) qs;
        if (!(lane & 1)) blk[66 + i0 / 4] = (uint8_t) (qh | (other << 4));
    } else if (V == 4) {
        *(uint16_t *) (blk + 2 + i0 / 2) = (uint16_t) qs;
        blk[66 + i0 / 4] = (uint8_t) qh;
    } else {
        *(uint16_t *) (blk + 2 + i0 / 2) = (uint16_t) qs;
        *(uint16_t *) (blk + 2 + i0 / 2 + 2) = (uint16_t) (qs >> 16);
        *(uint16_t *) (blk + 66 + i0 / 4) = (uint16_t) qh;
    }
}

static int launch_batch(RowBatch & bt, hipStream_t st) {
    bt.row_base[0] = 0;
    for (int k = 0; k < bt.n_jobs; ++k) bt.row_base[k + 1] = bt.row_base[k] + (bt.job[k].n_rows > 0 ? bt.job[k].n_rows : 0);
    const int n_rows = bt.row_base[bt.n_jobs];
    if (n_rows <= 0) return 0;
    const dim3 grid((unsigned) ((n_rows + ROW_WAVES - 1) / ROW_WAVES)), block(64 * ROW_WAVES);
    switch (bt.job[0].D) {
    case 128: hipLaunchKernelGGL(rows_kernel<2>, grid, block, 0, st, bt); break;
    case 256: hipLaunchKernelGGL(rows_kernel<4>, grid, block, 0, st, bt); break;
    case 512: hipLaunchKernelGGL(rows_kernel<8>, grid, block, 0, st, bt); break;
    default: return SJK_ERR_UNSUPPORTED;
    }
    return SJK_CHECK_LAUNCH();
}

static int launch_rows(const RowJob & j, hipStream_t st) {
    RowBatch bt = {};
    bt.job[0] = j;
    bt.n_jobs = 1;
    return launch_batch(bt, st);
}

static float rot_scale(int D) { return 1.0f / __builtin_sqrtf((float) D); }

// ---- unstage: one thread per value (sj_kvarn.h:1249-1260, 1276-1284) ----
__global__ void unstage_kernel(int staging, const uint8_t * src, size_t src_row_bytes, float * x, int D, int n_rows) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) n_rows * D) return;
    const size_t r = i / (size_t) D;
    const int e = (int) (i % (size_t) D);
    const uint8_t * row = src + r * src_row_bytes;
    if (staging == SJKVARN_STAGING_F16) {
        x[i] = f16_to_f32((uint16_t) (row[2 * e] | (row[2 * e + 1] << 8)));
        return;
    }
    const uint8_t * blk = row + (size_t) (e >> 7) * SJKVARN_TQ6_BLOCK_BYTES;
    const int jx = e & 127;
    const int code = ((blk[2 + (jx >> 1)] >> (4 * (jx & 1))) & 15) | (((blk[66 + (jx >> 2)] >> (2 * (jx & 3))) & 3) << 4);
    x[i] = xmul(tq6_cent(code), f16_to_f32((uint16_t) (blk[0] | (blk[1] << 8))));
}

// ---- decode: one thread per (record, token, channel) (sj_kvarn.h:1178-1207) ----
SJK_DEV float code_value(const sj_kvarn_layout & l, const uint8_t * rec, int t, int d, int is_v) {
    const int bits = is_v ? l.bits_v : l.bits_k;
    const uint8_t * payload = rec + (is_v ? l.v_payload : l.k_payload);
    if (l.body == SJKVARN_BODY_TRELLIS) return f16_to_f32(codebook(bits, is_v)[trellis_window(payload, bits, d, t)]);
    return (float) get_code(payload, code_bit(l, t, d, is_v), bits);
}

__global__ void decode_kernel(sj_kvarn_layout l, const uint8_t * body, int n_rec, float * out_k, float * out_v) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) n_rec * l.G * l.D) return;
    const int d = (int) (i % (size_t) l.D);
    const size_t rt = i / (size_t) l.D;
    const int t = (int) (rt % (size_t) l.G);
    const uint8_t * rec = body + (rt / (size_t) l.G) * l.bytes;
    const uint32_t ci = (uint32_t) k_ch_idx(l, d);
    out_k[i] = dequant_x(code_value(l, rec, t, d, 0), get_half(rec, l.k_scale + 2u * ci), get_half(rec, l.k_zero + 2u * ci),
                         get_half(rec, l.k_tok + 2u * (uint32_t) t));
    out_v[i] = dequant_x(code_value(l, rec, t, d, 1), get_half(rec, l.v_scale + 2u * (uint32_t) t),
                         get_half(rec, l.v_zero + 2u * (uint32_t) t), get_half(rec, l.v_ch + 2u * (uint32_t) v_ch_idx(l, d)));
}

// Gather / scatter of device byte runs (the sequence state stream: sink, records and ring rows of every layer
// to or from one staging buffer). Workgroups stride over the runs; the run descriptor is wave-uniform.
__global__ __launch_bounds__(256) void copy_runs_kernel(const CopyRun * runs, int n) {
    for (int r = (int) blockIdx.x; r < n; r += (int) gridDim.x) {
        const CopyRun R = runs[r];
        const uint64_t al = R.src | R.dst | R.bytes;
        if ((al & 15u) == 0) {
            const uint4 * s4 = (const uint4 *) R.src;
            uint4 * d4 = (uint4 *) R.dst;
            for (uint64_t i = threadIdx.x; i < R.bytes / 16u; i += blockDim.x) d4[i] = s4[i];
        } else if ((al & 3u) == 0) {
            const uint32_t * s1 = (const uint32_t *) R.src;
            uint32_t * d1 = (uint32_t *) R.dst;
            for (uint64_t i = threadIdx.x; i < R.bytes / 4u; i += blockDim.x) d1[i] = s1[i];
        } else {
            const uint8_t * s1 = (const uint8_t *) R.src;
            uint8_t * d1 = (uint8_t *) R.dst;
            for (uint64_t i = threadIdx.x; i < R.bytes; i += blockDim.x) d1[i] = s1[i];
        }
    }
}

int sjk_copy_runs(const CopyRun * d_runs, int n, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(copy_runs_kernel, dim3((unsigned) (n < 2048 ? n : 2048)), dim3(256), 0, stream, d_runs, n);
    return SJK_CHECK_LAUNCH();
}

// Zero the dst range of every run (src unused): the truncation / reset scrub of all layers in one launch
__global__ __launch_bounds__(256) void zero_runs_kernel(const CopyRun * runs, int n) {
    for (int r = (int) blockIdx.x; r < n; r += (int) gridDim.x) {
        const CopyRun R = runs[r];
        if (((R.dst | R.bytes) & 15u) == 0) {
            uint4 * d4 = (uint4 *) R.dst;
            for (uint64_t i = threadIdx.x; i < R.bytes / 16u; i += blockDim.x) d4[i] = uint4{0u, 0u, 0u, 0u};
        } else {
            uint8_t * d1 = (uint8_t *) R.dst;
            for (uint64_t i = threadIdx.x; i < R.bytes; i += blockDim.x) d1[i] = 0;
        }
    }
}

// Words carried in the kernel arguments, so the caller's host copy may change as soon as the launch returns
__global__ __launch_bounds__(256) void set_words_kernel(uint32_t * dst, const WordBatch w) {
    for (uint32_t i = threadIdx.x; i < w.n; i += 256) dst[i] = w.v[i];
}

int sjk_set_words(uint32_t * d_dst, const uint32_t * host, uint32_t n, hipStream_t stream) {
    WordBatch w;
    for (uint32_t o = 0; o < n; o += WORD_BATCH) {
        w.n = n - o < WORD_BATCH ? n - o : WORD_BATCH;
        for (uint32_t i = 0; i < w.n; ++i) w.v[i] = host[o + i];
        hipLaunchKernelGGL(set_words_kernel, dim3(1), dim3(256), 0, stream, d_dst + o, w);
        if (hipPeekAtLastError() != hipSuccess) return SJK_ERR_DEVICE;
    }
    return 0;
}

int sjk_zero_runs(const CopyRun * d_runs, int n, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(zero_runs_kernel, dim3((unsigned) (n < 2048 ? n : 2048)), dim3(256), 0, stream, d_runs, n);
    return SJK_CHECK_LAUNCH();
}

}  // namespace sjk

using namespace sjk;

namespace sjk {
// fp16 staging of rows of any width: one thread per value (sj_kvarn.h:1266-1271)
__global__ void stage_f16_kernel(const float * x, uint8_t * dst, int D, size_t dst_row_bytes, int n_rows) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) n_rows * (size_t) D) return;
    const size_t r = i / (size_t) D, e = i % (size_t) D;
    *(uint16_t *) (dst + r * dst_row_bytes + 2 * e) = f32_to_f16(x[i]);
}
}  // namespace sjk

extern "C" int sjk_hip_stage(int staging, const float * d_x, uint8_t * d_dst, int D, size_t dst_row_bytes, int n_rows,
                             void * stream) {
    if (!d_x || !d_dst || n_rows < 0 || D <= 0 || (staging != SJKVARN_STAGING_TQ6_0 && staging != SJKVARN_STAGING_F16))
        return SJKVARN_ERR_ARG;
    if (!n_rows) return 0;
    if (D != 128 && D != 256 && D != 512) {
        hipStream_t st = (hipStream_t) stream;
        if (staging == SJKVARN_STAGING_F16) {
            const size_t n = (size_t) n_rows * (size_t) D;
            hipLaunchKernelGGL(stage_f16_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, d_x, d_dst, D,
                               dst_row_bytes, n_rows);
            return SJK_CHECK_LAUNCH();
        }
        // tq6_0: the D / 128 whole blocks of each row (the reference quantizes n / 128 blocks), as rows of 128
        const int nb = D / SJKVARN_TQ6_QK;
        if (!nb) return 0;
        for (int r = 0; r < n_rows; ++r) {
            const bool packed = dst_row_bytes == (size_t) nb * SJKVARN_TQ6_BLOCK_BYTES && D % SJKVARN_TQ6_QK == 0;
            RowJob j = {};
            j.kind = 0; j.D = SJKVARN_TQ6_QK; j.rotate = 0; j.rot_scale = rot_scale(SJKVARN_TQ6_QK);
            j.n_rows = packed ? nb * n_rows : nb;
            j.x = d_x + (size_t) r * D; j.dst = d_dst + (size_t) r * dst_row_bytes;
            j.dst_row_bytes = SJKVARN_TQ6_BLOCK_BYTES; j.out_mode = OUT_TQ6;
            const int rc = launch_rows(j, st);
            if (rc || packed) return rc;
        }
        return 0;
    }
    RowJob j = {};
    j.kind = 0; j.D = D; j.n_rows = n_rows; j.rotate = 0; j.rot_scale = rot_scale(D);
    j.x = d_x; j.dst = d_dst; j.dst_row_bytes = dst_row_bytes;
    j.out_mode = staging == SJKVARN_STAGING_F16 ? OUT_F16 : OUT_TQ6;
    return launch_rows(j, (hipStream_t) stream);
}

namespace sjk {

// Hadamard of rows of any power-of-two length n (sj_kvarn.h:735-752) outside the row kernel's widths: stage h pairs
// element j with j + h (j in the lower half of its 2h block) as a + b, a - b, stages in ascending h, then one
// multiply by s. The order of the stages, not the order of the pairs inside a stage, fixes every value, so
// these are bit-identical to the reference's loop.
constexpr int HD_LDS_MAX = 8192;          // rows up to 32 KB go through LDS, one workgroup per row

__global__ __launch_bounds__(256) void hadamard_lds_kernel(float * x, int n, float s) {
    extern __shared__ float t[];
    float * row = x + (size_t) blockIdx.x * (size_t) n;
    for (int i = (int) threadIdx.x; i < n; i += 256) t[i] = row[i];
    __syncthreads();
    for (int h = 1; h < n; h <<= 1) {
        for (int k = (int) threadIdx.x; k < n / 2; k += 256) {
            const int j = (k / h) * 2 * h + (k % h);
            const float a = t[j], b = t[j + h];
            t[j] = xadd(a, b);
            t[j + h] = xsub(a, b);
        }
        __syncthreads();
    }
    for (int i = (int) threadIdx.x; i < n; i += 256) row[i] = xmul(t[i], s);
}

// one stage of longer rows in global memory: pair k of the n_rows * n / 2 pairs
__global__ __launch_bounds__(256) void hadamard_stage_kernel(float * x, int n, int h, size_t n_pairs) {
    const size_t k = (size_t) blockIdx.x * 256u + threadIdx.x;
    if (k >= n_pairs) return;
    const size_t row = k / (size_t) (n / 2), kk = k % (size_t) (n / 2);
    const size_t j = row * (size_t) n + (kk / (size_t) h) * 2u * (size_t) h + kk % (size_t) h;
    const float a = x[j], b = x[j + (size_t) h];
    x[j] = xadd(a, b);
    x[j + (size_t) h] = xsub(a, b);
}

// one stage along the rows of a [n_blocks * n][cols] matrix (each column's n-blocks are the vectors): pair k of the
// n_blocks * n / 2 * cols pairs, column fastest (adjacent threads, adjacent columns)
__global__ __launch_bounds__(256) void hadamard_cols_stage_kernel(float * x, int n, int h, int cols, size_t n_pairs) {
    const size_t k = (size_t) blockIdx.x * 256u + threadIdx.x;
    if (k >= n_pairs) return;
    const size_t c = k % (size_t) cols, rest = k / (size_t) cols;
    const size_t blk = rest / (size_t) (n / 2), kk = rest % (size_t) (n / 2);
    const size_t j = blk * (size_t) n + (kk / (size_t) h) * 2u * (size_t) h + kk % (size_t) h;
    float * pa = x + j * (size_t) cols + c;
    float * pb = pa + (size_t) h * (size_t) cols;
    const float a = *pa, b = *pb;
    *pa = xadd(a, b);
    *pb = xsub(a, b);
}

__global__ __launch_bounds__(256) void scale_kernel(float * x, size_t n, float s) {
    const size_t i = (size_t) blockIdx.x * 256u + threadIdx.x;
    if (i < n) x[i] = xmul(x[i], s);
}

}  // namespace sjk

// Rotation folded into projection weights. Output side (W_q, W_k, W_v, their biases): [n_heads * D][cols], each
// column's head blocks rotated, i.e. the per-head rotation applied from the left, W' = blockdiag(R) W. Input side
// (W_o): [rows][n_heads * D], each row's head segments rotated, W' = W blockdiag(R) (R = H / sqrt(D) is
// symmetric and its own inverse) - sjk_hip_rotate over rows x n_heads segments of D.
extern "C" int sjk_hip_fold_rotation_out(float * d_w, int n_heads, int D, int cols, void * stream) {
    if (!d_w || n_heads < 0 || cols < 0 || D <= 0 || (D & (D - 1))) return SJKVARN_ERR_ARG;
    if (!n_heads || !cols) return 0;
    hipStream_t st = (hipStream_t) stream;
    const size_t pairs = (size_t) n_heads * (size_t) (D / 2) * (size_t) cols, all = (size_t) n_heads * D * (size_t) cols;
    for (int h = 1; h < D; h <<= 1) {
        hipLaunchKernelGGL(hadamard_cols_stage_kernel, dim3((unsigned) ((pairs + 255) / 256)), dim3(256), 0, st, d_w, D,
                           h, cols, pairs);
        if (SJK_CHECK_LAUNCH()) return SJK_ERR_DEVICE;
    }
    hipLaunchKernelGGL(scale_kernel, dim3((unsigned) ((all + 255) / 256)), dim3(256), 0, st, d_w, all, rot_scale(D));
    return SJK_CHECK_LAUNCH();
}

extern "C" int sjk_hip_rotate(float * d_x, int n_rows, int D, void * stream);

extern "C" int sjk_hip_fold_rotation_in(float * d_w, int rows, int n_heads, int D, void * stream) {
    if (!d_w || rows < 0 || n_heads < 0 || D <= 0 || (D & (D - 1))) return SJKVARN_ERR_ARG;
    if ((size_t) rows * (size_t) n_heads > (size_t) 0x7fffffff) return SJKVARN_ERR_ARG;
    return sjk_hip_rotate(d_w, rows * n_heads, D, stream);
}

extern "C" int sjk_hip_rotate(float * d_x, int n_rows, int D, void * stream) {
    if (!d_x || n_rows < 0 || D <= 0 || (D & (D - 1))) return SJKVARN_ERR_ARG;
    if (!n_rows) return 0;
    hipStream_t st = (hipStream_t) stream;
    if (D == 128 || D == 256 || D == 512) {
        RowJob j = {};
        j.kind = 0; j.D = D; j.n_rows = n_rows; j.rotate = 1; j.rot_scale = rot_scale(D);
        j.x = d_x; j.dst = (uint8_t *) d_x; j.dst_row_bytes = (size_t) D * 4; j.out_mode = OUT_F32;
        return launch_rows(j, st);
    }
    const float s = rot_scale(D);
    if (D <= HD_LDS_MAX) {
        hipLaunchKernelGGL(hadamard_lds_kernel, dim3((unsigned) n_rows), dim3(256), (size_t) D * 4, st, d_x, D, s);
        return SJK_CHECK_LAUNCH();
    }
    const size_t pairs = (size_t) n_rows * (size_t) (D / 2), all = (size_t) n_rows * (size_t) D;
    for (int h = 1; h < D; h <<= 1) {
        hipLaunchKernelGGL(hadamard_stage_kernel, dim3((unsigned) ((pairs + 255) / 256)), dim3(256), 0, st, d_x, D, h, pairs);
        if (SJK_CHECK_LAUNCH()) return SJK_ERR_DEVICE;
    }
    hipLaunchKernelGGL(scale_kernel, dim3((unsigned) ((all + 255) / 256)), dim3(256), 0, st, d_x, all, s);
    return SJK_CHECK_LAUNCH();
}

static RowJob store_job(const sjk_hip_view * v, uint32_t pos0, uint32_t n_pos, const float * d_k, const float * d_v,
                        int rotate) {
    RowJob j = {};
    j.kind = 1; j.D = v->lay.D; j.n_rows = (int) n_pos * v->n_head_kv * 2; j.rotate = rotate ? 1 : 0;
    j.rot_scale = rot_scale(v->lay.D);
    j.k = d_k; j.v = d_v; j.sink = v->sink; j.ring = v->ring;
    j.pos0 = pos0; j.S = v->S; j.cap = v->cap; j.H = v->n_head_kv; j.sink_type = v->sink_type;
    j.staging = v->staging; j.stage_bytes = v->stage_bytes;
    return j;
}

extern "C" int sjk_hip_layer_store(const sjk_hip_view * v, uint32_t pos0, uint32_t n_pos, const float * d_k,
                                   const float * d_v, int rotate, void * stream) {
    if (!v || !d_k || !d_v || !v->sink || !v->ring) return SJKVARN_ERR_ARG;
    return launch_rows(store_job(v, pos0, n_pos, d_k, d_v, rotate), (hipStream_t) stream);
}

extern "C" int sjk_hip_layer_store_dyn(const sjk_hip_view * v, const int32_t * d_desc, uint32_t n_pos, const float * d_k,
                                       const float * d_v, int rotate, void * stream) {
    if (!v || !d_desc || !d_k || !d_v || !v->sink || !v->ring) return SJKVARN_ERR_ARG;
    RowJob j = store_job(v, 0, n_pos, d_k, d_v, rotate);
    j.pos_desc = d_desc;
    return launch_rows(j, (hipStream_t) stream);
}

extern "C" int sjk_hip_store_batch(const sjk_hip_store_job * jobs, int n_jobs, uint32_t n_pos, int rotate, void * stream) {
    if (n_jobs < 0 || (n_jobs > 0 && !jobs)) return SJKVARN_ERR_ARG;
    for (int k = 0; k < n_jobs; ++k)
        if (!jobs[k].d_k || !jobs[k].d_v || !jobs[k].v.sink || !jobs[k].v.ring || jobs[k].v.lay.D != jobs[0].v.lay.D)
            return SJKVARN_ERR_ARG;
    for (int k0 = 0; k0 < n_jobs; k0 += ROW_MAXJ) {
        RowBatch bt = {};
        bt.n_jobs = n_jobs - k0 < ROW_MAXJ ? n_jobs - k0 : ROW_MAXJ;
        for (int k = 0; k < bt.n_jobs; ++k) {
            const sjk_hip_store_job & J = jobs[k0 + k];
            bt.job[k] = store_job(&J.v, J.pos0, n_pos, J.d_k, J.d_v, rotate);
        }
        const int rc = launch_batch(bt, (hipStream_t) stream);
        if (rc) return rc;
    }
    return 0;
}

extern "C" int sjk_hip_unstage(int staging, const uint8_t * d_src, size_t src_row_bytes, float * d_x, int D, int n_rows,
                               void * stream) {
    if (!d_src || !d_x || n_rows < 0 || D <= 0 || (staging == SJKVARN_STAGING_TQ6_0 && D % 128)) return SJKVARN_ERR_ARG;
    const size_t n = (size_t) n_rows * D;
    if (!n) return 0;
    hipLaunchKernelGGL(unstage_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, (hipStream_t) stream, staging,
                       d_src, src_row_bytes, d_x, D, n_rows);
    return SJK_CHECK_LAUNCH();
}

extern "C" int sjk_hip_decode(const sj_kvarn_layout * l, const uint8_t * d_body, int n_rec, float * d_out_k,
                              float * d_out_v, void * stream) {
    if (!l || !d_body || !d_out_k || !d_out_v || n_rec < 0) return SJKVARN_ERR_ARG;
    const size_t n = (size_t) n_rec * l->G * l->D;
    if (!n) return 0;
    hipLaunchKernelGGL(decode_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, (hipStream_t) stream, *l, d_body,
                       n_rec, d_out_k, d_out_v);
    return SJK_CHECK_LAUNCH();
}

namespace sjk {

// ---- record_scores / record_accum_v (sj_kvarn.h:1288-1311): sequential fp32 as in the reference ----
SJK_DEV float decode_k_at(const sj_kvarn_layout & l, const uint8_t * rec, int t, int d) {
    const uint32_t ci = (uint32_t) k_ch_idx(l, d);
    return dequant_x(code_value(l, rec, t, d, 0), get_half(rec, l.k_scale + 2u * ci), get_half(rec, l.k_zero + 2u * ci),
                     get_half(rec, l.k_tok + 2u * (uint32_t) t));
}

SJK_DEV float decode_v_at(const sj_kvarn_layout & l, const uint8_t * rec, int t, int d) {
    return dequant_x(code_value(l, rec, t, d, 1), get_half(rec, l.v_scale + 2u * (uint32_t) t),
                     get_half(rec, l.v_zero + 2u * (uint32_t) t), get_half(rec, l.v_ch + 2u * (uint32_t) v_ch_idx(l, d)));
}

__global__ void record_scores_kernel(sj_kvarn_layout l, const uint8_t * rec, const float * q, int n, float * scores) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    float s = 0.0f;
    for (int d = 0; d < l.D; ++d) s = s + q[d] * decode_k_at(l, rec, t, d);
    scores[t] = s;
}

__global__ void record_accum_kernel(sj_kvarn_layout l, const uint8_t * rec, const float * w, int n, float * acc) {
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= l.D) return;
    float a = acc[d];
    for (int t = 0; t < n; ++t) a = a + w[t] * decode_v_at(l, rec, t, d);
    acc[d] = a;
}

}  // namespace sjk

extern "C" int sjk_hip_record_scores(const sj_kvarn_layout * l, const uint8_t * d_rec, const float * d_q, int n,
                                     float * d_scores, void * stream) {
    if (!l || !d_rec || !d_q || !d_scores || n < 0 || n > l->G) return SJKVARN_ERR_ARG;
    if (!n) return 0;
    hipLaunchKernelGGL(sjk::record_scores_kernel, dim3((unsigned) ((n + 127) / 128)), dim3(128), 0, (hipStream_t) stream,
                       *l, d_rec, d_q, n, d_scores);
    return SJK_CHECK_LAUNCH();
}

extern "C" int sjk_hip_record_accum_v(const sj_kvarn_layout * l, const uint8_t * d_rec, const float * d_w, int n,
                                      float * d_acc, void * stream) {
    if (!l || !d_rec || !d_w || !d_acc || n < 0 || n > l->G) return SJKVARN_ERR_ARG;
    hipLaunchKernelGGL(sjk::record_accum_kernel, dim3((unsigned) ((l->D + 127) / 128)), dim3(128), 0, (hipStream_t) stream,
                       *l, d_rec, d_w, n, d_acc);
    return SJK_CHECK_LAUNCH();
}
