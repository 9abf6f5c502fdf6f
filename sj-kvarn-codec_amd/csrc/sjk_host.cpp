// sjk_host.cpp - host side of libsjk.so: the sj_kvarn.h API (same names and argument meaning,
// reference sj_kvarn.h:177-453) over device-resident caches and the HIP kernels.
//
// Integer bookkeeping (layout offsets, journal policy, ring slots, pool free list, state-stream
// headers) runs on the host as in the reference; every byte of codec output (records, staging rows,
// decoded rows, scores) is produced by a HIP kernel. The void codec calls of the reference API take
// host arrays: the free functions copy them to device buffers of their own call, the layer calls to
// the layer's workspace, launch, and copy the result back (synchronous). There is no CPU path: a HIP
// failure inside a void call (which has no status to return) aborts with a message. There is no
// process-wide mutable state: every buffer belongs to a call or to a cache object.
#include <hip/hip_runtime.h>

#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "../../include/sjk.h"
#include "../../include/sjk_tables.h"
#include "sjk_dev.h"

namespace {

thread_local char g_err[256] = "";        // the calling thread's last HIP error text (sjk_last_error)

int hip_fail(hipError_t e, const char * what) {
    snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
    return SJK_ERR_DEVICE;
}

#define HIP_TRY(call)                                         \
    do {                                                      \
        const hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return hip_fail(e_, #call);     \
    } while (0)

[[noreturn]] void die(const char * fn, const char * what) {
    fprintf(stderr, "libsjk: %s: %s\n", fn, what);
    abort();
}

void must(int rc, const char * fn) {
    if (rc) die(fn, rc == SJK_ERR_DEVICE ? g_err : sj_kvarn_strerror(rc));
}

void must_hip(hipError_t e, const char * fn) {
    if (e != hipSuccess) die(fn, hipGetErrorString(e));
}

// Device buffers of the host-array calls: a set of four per host thread and device, grown on demand and kept until
// the process ends (a hipFree per call would wait for the whole device). A call's copies back are synchronous, so
// its buffers are free again when it returns.
constexpr int CALL_BUFS = 4;
thread_local void * t_buf[CALL_BUFS] = {};
thread_local size_t t_cap[CALL_BUFS] = {};
thread_local int t_dev[CALL_BUFS] = {-1, -1, -1, -1};

struct CallBufs {
    int n = 0;
    const char * fn;
    explicit CallBufs(const char * f) : fn(f) {}
    template <typename T> T * get(size_t bytes) {
        if (n >= CALL_BUFS) die(fn, "more device buffers than a host-array call has");
        int dev = 0;
        must_hip(hipGetDevice(&dev), fn);
        if (t_cap[n] < bytes || t_dev[n] != dev || !t_buf[n]) {
            if (t_buf[n] && t_dev[n] == dev) (void) hipFree(t_buf[n]);
            const size_t want = bytes > 4096 ? bytes : 4096;
            must_hip(hipMalloc(&t_buf[n], want), fn);
            t_cap[n] = want;
            t_dev[n] = dev;
        }
        return (T *) t_buf[n++];
    }
};

void h2d(void * d, const void * h, size_t n, const char * fn) { if (n) must_hip(hipMemcpy(d, h, n, hipMemcpyHostToDevice), fn); }
void d2h(void * h, const void * d, size_t n, const char * fn) { if (n) must_hip(hipMemcpy(h, d, n, hipMemcpyDeviceToHost), fn); }
// the host-array layer calls launch on the null stream and wait for it (not for the rest of the device)
void null_sync(const char * fn) { must_hip(hipStreamSynchronize(nullptr), fn); }

uint64_t fnv1a(const void * p, size_t n, uint64_t h) {
    const uint8_t * b = (const uint8_t *) p;
    for (size_t i = 0; i < n; ++i) { h ^= b[i]; h *= 1099511628211ull; }
    return h;
}
constexpr uint64_t FNV0 = 1469598103934665603ull;

bool frag_side(const sj_kvarn_layout * l, int bits) {
    return l->body == SJKVARN_BODY_SCALAR && bits == 4 && l->D % 16 == 0 && l->G % 16 == 0;
}

// ---------------------------------------------------------------------------------------------------
// runtime of a cache object
// ---------------------------------------------------------------------------------------------------

constexpr int RT_STORE_STREAMS = 4;
struct StateJob;

// The library's runtime of one cache object (a layer made by sj_kvarn_layer_init, or a sequence, kept with its
// first layer), reached through the layer's vstage field and freed with the object:
//   * st: the object's own stream (non-blocking) for its commits and state transfers, xst for the host copies of
//     an asynchronous state save or restore, so that commits do not queue behind them;
//   * the streams the object's device stores used (sjk_hip_seq_store and _batch) since its last host-synchronous
//     commit: such a commit waits for events on them, not for the whole device (more than four streams: the
//     whole device);
//   * the device run table of truncation scrubs, sized at init (n_layers x (groups + 3) runs: every record
//     group, the sink range and two ring ranges per layer), so that a truncation allocates nothing;
//   * the state transfer buffers (two 32 MB device stages and pinned host buffers with their run tables) and the
//     device snapshot of an asynchronous save or restore, allocated by the first call that needs them and kept.
struct Rt {
    hipStream_t st = nullptr, xst = nullptr;
    hipEvent_t done = nullptr;
    hipEvent_t mark[RT_STORE_STREAMS + 1] = {};     // the last one marks the null stream
    hipStream_t store_st[RT_STORE_STREAMS] = {};
    int n_store = 0;
    bool store_many = false;
    sjk::CopyRun * d_runs = nullptr;
    size_t max_runs = 0;
    uint8_t * dstage[2] = {};
    sjk::CopyRun * druns[2] = {};
    uint8_t * hpin[2] = {};
    sjk::CopyRun * hruns[2] = {};
    hipEvent_t xev[2] = {};
    bool xfer_ready = false;
    uint8_t * snap = nullptr;
    size_t snap_cap = 0;
    StateJob * job = nullptr;
};

Rt * rt_of(const sj_kvarn_layer * L) { return L ? (Rt *) (void *) L->vstage : nullptr; }
Rt * rt_of(const sj_kvarn_seq * s) { return s && s->layers && s->n_layers > 0 ? rt_of(&s->layers[0]) : nullptr; }

void rt_destroy(Rt * r);

Rt * rt_create(size_t max_runs) {
    Rt * r = new (std::nothrow) Rt();
    if (!r) return nullptr;
    bool ok = hipStreamCreateWithFlags(&r->st, hipStreamNonBlocking) == hipSuccess &&
              hipStreamCreateWithFlags(&r->xst, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&r->done, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; ok && i <= RT_STORE_STREAMS; ++i) ok = hipEventCreateWithFlags(&r->mark[i], hipEventDisableTiming) == hipSuccess;
    r->max_runs = max_runs;
    if (ok) ok = hipMalloc((void **) &r->d_runs, (max_runs ? max_runs : 1) * sizeof(sjk::CopyRun)) == hipSuccess;
    if (!ok) { rt_destroy(r); return nullptr; }
    return r;
}

// a device store into the object was enqueued on stream st
void rt_note_store(Rt * r, hipStream_t st) {
    if (!r) return;
    for (int i = 0; i < r->n_store; ++i) if (r->store_st[i] == st) return;
    if (r->n_store < RT_STORE_STREAMS) r->store_st[r->n_store++] = st;
    else r->store_many = true;
}

// make stream st wait for the work already enqueued on the null stream and on the streams the object's stores used
int rt_after_stores(Rt * r, hipStream_t st) {
    if (r->store_many) {
        HIP_TRY(hipDeviceSynchronize());
    } else {
        HIP_TRY(hipEventRecord(r->mark[RT_STORE_STREAMS], nullptr));
        HIP_TRY(hipStreamWaitEvent(st, r->mark[RT_STORE_STREAMS], 0));
        for (int i = 0; i < r->n_store; ++i) {
            if (!r->store_st[i]) continue;            // the null stream: done above
            HIP_TRY(hipEventRecord(r->mark[i], r->store_st[i]));
            HIP_TRY(hipStreamWaitEvent(st, r->mark[i], 0));
        }
    }
    return 0;
}

// wait on the host for the work enqueued on st; the object's earlier stores are then complete
int rt_wait(Rt * r, hipStream_t st) {
    HIP_TRY(hipEventRecord(r->done, st));
    HIP_TRY(hipEventSynchronize(r->done));
    r->n_store = 0;
    r->store_many = false;
    return 0;
}

// the state transfer buffers, on first use
int rt_xfer_buffers(Rt * r);

}  // namespace

extern "C" {

const char * sjk_last_error(void) { return g_err; }

}  // extern "C"

namespace sjk {
// the text sjk_last_error() returns on this thread (for refusals that are not HIP errors)
void set_error(const char * what) { snprintf(g_err, sizeof(g_err), "%s", what); }
}  // namespace sjk

extern "C" {

// ---------------------------------------------------------------------------------------------------
// fp16 (sj_kvarn.h:693-731): host scalar helpers for engines that write rows themselves
// ---------------------------------------------------------------------------------------------------

uint16_t sj_kvarn_f32_to_f16(float f) {
    uint32_t w;
    memcpy(&w, &f, 4);
    const uint32_t sign = (w >> 16) & 0x8000u, a = w & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t) (sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t) (sign | 0x7C00u);
    if (a >= 0x38800000u) return (uint16_t) (sign | ((a + 0x0FFFu + ((a >> 13) & 1u) - 0x38000000u) >> 13));
    const uint32_t e = a >> 23;
    if (e < 102u) return (uint16_t) sign;
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t) (sign | q);
}

float sj_kvarn_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3FFu;
    uint32_t w;
    float f;
    if (e == 31u) w = sign | 0x7F800000u | (m << 13);
    else if (e != 0u) w = sign | ((e + 112u) << 23) | (m << 13);
    else { f = (float) m * 0x1p-24f; return sign ? -f : f; }
    memcpy(&f, &w, 4);
    return f;
}

// ---------------------------------------------------------------------------------------------------
// record layout (sj_kvarn.h:763-849)
// ---------------------------------------------------------------------------------------------------

int sj_kvarn_body_resolve(int body, int bits_k, int bits_v) {
    if (body != SJKVARN_BODY_AUTO) return body;
    const bool t = (bits_k == 2 || bits_k == 3) && (bits_v == 2 || bits_v == 3) && bits_v <= bits_k;
    return t ? SJKVARN_BODY_TRELLIS : SJKVARN_BODY_SCALAR;
}

int sj_kvarn_layout_init(sj_kvarn_layout * l, int D, int G, int bits_k, int bits_v, int body) {
    if (D < 32 || (D & (D - 1)) || G <= 0 || G % 16) return -1;
    if (bits_k < 2 || bits_k > 4 || bits_v < 2 || bits_v > 4) return -2;
    if (body != SJKVARN_BODY_SCALAR && body != SJKVARN_BODY_TRELLIS) return -3;
    if (body == SJKVARN_BODY_TRELLIS &&
        (bits_k == 4 || bits_v == 4 || bits_v > bits_k || G != SJKVARN_TRELLIS_SEQ || D % SJKVARN_TRELLIS_SEQ))
        return -4;
    l->D = D; l->G = G; l->bits_k = bits_k; l->bits_v = bits_v; l->body = body;
    uint32_t off = 0;
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

size_t sj_kvarn_record_bytes(int D, int G, int bits_k, int bits_v) {
    return (size_t) G * D * bits_k / 8 + (size_t) G * D * bits_v / 8 + 6 * (size_t) D + 6 * (size_t) G;
}

double sj_kvarn_body_bits_per_element(const sj_kvarn_layout * l) {
    return 8.0 * (double) l->bytes / (2.0 * (double) l->D * (double) l->G);
}

uint32_t sj_kvarn_code_bit(const sj_kvarn_layout * l, int t, int d, int is_v) {
    const int bits = is_v ? l->bits_v : l->bits_k;
    if (l->body == SJKVARN_BODY_TRELLIS) return ((uint32_t) d * (uint32_t) l->G + (uint32_t) t) * (uint32_t) bits;
    if (!frag_side(l, bits)) return ((uint32_t) t * (uint32_t) l->D + (uint32_t) d) * (uint32_t) bits;
    const int a = is_v ? d : t, b = is_v ? t : d, aa = a & 15, bb = b & 15;
    const uint32_t tile = (uint32_t) ((t >> 4) * (l->D / 16) + (d >> 4));
    const uint32_t word = tile * 32u + (uint32_t) (4 * (aa & 7) + ((bb >> 1) & 3));
    const uint32_t nib = (uint32_t) ((aa >> 3) + 2 * (bb >> 3) + 4 * (bb & 1));
    return word * 32u + nib * 4u;
}

int sj_kvarn_k_ch_idx(const sj_kvarn_layout * l, int d) {
    if (!frag_side(l, l->bits_k)) return d;
    const int c = d >> 4, dd = d & 15, jj = dd >> 1;
    return (jj & 3) * (l->D / 4) + c * 4 + (jj >> 2) * 2 + (dd & 1);
}

int sj_kvarn_v_ch_idx(const sj_kvarn_layout * l, int d) {
    if (!frag_side(l, l->bits_v)) return d;
    return (d & 7) * (l->D / 8) + (d >> 4) * 2 + ((d >> 3) & 1);
}

// the reference's host workspace figure (sj_kvarn.h:906-937), reported for ABI compatibility
size_t sj_kvarn_seal_workspace_bytes(const sj_kvarn_layout * l) {
    const size_t DG = (size_t) l->D * (size_t) l->G, R = (size_t) (l->D > l->G ? l->D : l->G);
    const size_t sizes[14] = {4 * DG, 4 * DG, 4 * R, 4 * R, 4 * R, 4 * R, 8 * R, 8 * R, 4 * 128, 4 * 512, 4 * 64, 4 * 64,
                              128, 128 * 64};
    size_t at = 0;
    for (size_t s : sizes) at = (at + s + 7u) & ~(size_t) 7u;
    return at;
}

size_t sj_kvarn_stage_row_bytes(int staging, int D) {
    return staging == SJKVARN_STAGING_F16 ? (size_t) D * 2 : (size_t) (D / SJKVARN_TQ6_QK) * SJKVARN_TQ6_BLOCK_BYTES;
}

// ---------------------------------------------------------------------------------------------------
// codec calls on host arrays (device round trip)
// ---------------------------------------------------------------------------------------------------

// Any power of two n (the reference's stages index past the end of x otherwise, sj_kvarn.h:735-752): other n
// leave x as it is.
void sj_kvarn_hadamard(float * x, int n) {
    if (n <= 0 || (n & (n - 1))) return;
    CallBufs b("sj_kvarn_hadamard");
    float * d = b.get<float>((size_t) n * 4);
    h2d(d, x, (size_t) n * 4, b.fn);
    must(sjk_hip_rotate(d, 1, n, nullptr), b.fn);
    d2h(x, d, (size_t) n * 4, b.fn);
}

void sj_kvarn_rotate_heads(float * x, int n_heads, int head_dim) {
    if (n_heads <= 0 || head_dim <= 0 || (head_dim & (head_dim - 1))) return;
    CallBufs b("sj_kvarn_rotate_heads");
    const size_t bytes = (size_t) n_heads * head_dim * 4;
    float * d = b.get<float>(bytes);
    h2d(d, x, bytes, b.fn);
    must(sjk_hip_rotate(d, n_heads, head_dim, nullptr), b.fn);
    d2h(x, d, bytes, b.fn);
}

// A layout the device seal is not built for (sjk_hip_supported: D 128 or 256, G 128) aborts with a message, as a
// device failure in any void call does: there is no status to return, no CPU path, and a record left unwritten
// would be taken for a sealed one.
void sj_kvarn_seal_group(const sj_kvarn_layout * l, const uint16_t * K, const uint16_t * V, size_t row_stride, int iters,
                         uint8_t * rec, void * work) {
    (void) work;
    if (!sjk_hip_supported(l)) {
        char what[160];
        snprintf(what, sizeof(what), "layout D=%d G=%d bits %d/%d is not supported by the HIP seal (D 128 or 256, "
                                     "G 128)", l->D, l->G, l->bits_k, l->bits_v);
        die("sj_kvarn_seal_group", what);
    }
    CallBufs b("sj_kvarn_seal_group");
    const size_t rows = (size_t) (l->G - 1) * row_stride + (size_t) l->D;
    uint16_t * dk = b.get<uint16_t>(rows * 2);
    uint16_t * dv = b.get<uint16_t>(rows * 2);
    uint8_t * dr = b.get<uint8_t>(l->bytes);
    h2d(dk, K, rows * 2, b.fn);
    h2d(dv, V, rows * 2, b.fn);
    must(sjk_hip_seal(l, dk, dv, row_stride, 1, 1, iters, dr, nullptr), b.fn);
    d2h(rec, dr, l->bytes, b.fn);
}

static void decode_row(const sj_kvarn_layout * l, const uint8_t * rec, int t, float * out, int is_v) {
    CallBufs b("sj_kvarn_decode_row");
    uint8_t * dr = b.get<uint8_t>(l->bytes);
    const size_t rows = (size_t) l->G * l->D * 4;
    float * dk = b.get<float>(rows);
    float * dv = b.get<float>(rows);
    h2d(dr, rec, l->bytes, b.fn);
    must(sjk_hip_decode(l, dr, 1, dk, dv, nullptr), b.fn);
    d2h(out, (is_v ? dv : dk) + (size_t) t * l->D, (size_t) l->D * 4, b.fn);
}

void sj_kvarn_decode_k_row(const sj_kvarn_layout * l, const uint8_t * rec, int t, float * out) { decode_row(l, rec, t, out, 0); }
void sj_kvarn_decode_v_row(const sj_kvarn_layout * l, const uint8_t * rec, int t, float * out) { decode_row(l, rec, t, out, 1); }

void sj_kvarn_tq6_quantize_row(const float * x, sj_kvarn_tq6_block * y, int n) {
    const int nb = n / SJKVARN_TQ6_QK;
    if (nb <= 0) return;
    CallBufs b("sj_kvarn_tq6_quantize_row");
    float * dx = b.get<float>((size_t) nb * SJKVARN_TQ6_QK * 4);
    uint8_t * dy = b.get<uint8_t>((size_t) nb * SJKVARN_TQ6_BLOCK_BYTES);
    h2d(dx, x, (size_t) nb * SJKVARN_TQ6_QK * 4, b.fn);
    // blocks are independent: the row is staged as nb rows of 128 values
    must(sjk_hip_stage(SJKVARN_STAGING_TQ6_0, dx, dy, SJKVARN_TQ6_QK, SJKVARN_TQ6_BLOCK_BYTES, nb, nullptr), b.fn);
    d2h(y, dy, (size_t) nb * SJKVARN_TQ6_BLOCK_BYTES, b.fn);
}

void sj_kvarn_tq6_dequantize_row(const sj_kvarn_tq6_block * y, float * x, int n) {
    const int nb = n / SJKVARN_TQ6_QK;
    if (nb <= 0) return;
    CallBufs b("sj_kvarn_tq6_dequantize_row");
    uint8_t * dy = b.get<uint8_t>((size_t) nb * SJKVARN_TQ6_BLOCK_BYTES);
    float * dx = b.get<float>((size_t) nb * SJKVARN_TQ6_QK * 4);
    h2d(dy, y, (size_t) nb * SJKVARN_TQ6_BLOCK_BYTES, b.fn);
    must(sjk_hip_unstage(SJKVARN_STAGING_TQ6_0, dy, SJKVARN_TQ6_BLOCK_BYTES, dx, SJKVARN_TQ6_QK, nb, nullptr), b.fn);
    d2h(x, dx, (size_t) nb * SJKVARN_TQ6_QK * 4, b.fn);
}

// any D (sjk_hip_stage takes every width: the row kernel for D in {128, 256, 512}, else a per-value fp16 kernel or
// tq6_0 rows of 128)
void sj_kvarn_stage_row(int staging, const float * x_rot, void * dst, int D) {
    if (staging == SJKVARN_STAGING_TQ6_0) { sj_kvarn_tq6_quantize_row(x_rot, (sj_kvarn_tq6_block *) dst, D); return; }
    if (D <= 0) return;
    CallBufs b("sj_kvarn_stage_row");
    const size_t ob = sj_kvarn_stage_row_bytes(staging, D);
    float * dx = b.get<float>((size_t) D * 4);
    uint8_t * dy = b.get<uint8_t>(ob);
    h2d(dx, x_rot, (size_t) D * 4, b.fn);
    must(sjk_hip_stage(staging, dx, dy, D, ob, 1, nullptr), b.fn);
    d2h(dst, dy, ob, b.fn);
}

void sj_kvarn_unstage_row(int staging, const void * src, float * x_rot, int D) {
    if (staging == SJKVARN_STAGING_TQ6_0) {
        sj_kvarn_tq6_dequantize_row((const sj_kvarn_tq6_block *) src, x_rot, D);
        return;
    }
    if (D <= 0) return;
    CallBufs b("sj_kvarn_unstage_row");
    const size_t ib = sj_kvarn_stage_row_bytes(staging, D);
    uint8_t * dy = b.get<uint8_t>(ib);
    float * dx = b.get<float>((size_t) D * 4);
    h2d(dy, src, ib, b.fn);
    must(sjk_hip_unstage(staging, dy, ib, dx, D, 1, nullptr), b.fn);
    d2h(x_rot, dx, (size_t) D * 4, b.fn);
}

void sj_kvarn_record_scores(const sj_kvarn_layout * l, const uint8_t * rec, const float * q, int n, float * scores) {
    if (n <= 0) return;
    CallBufs b("sj_kvarn_record_scores");
    uint8_t * dr = b.get<uint8_t>(l->bytes);
    float * dq = b.get<float>((size_t) l->D * 4);
    float * ds = b.get<float>((size_t) l->G * 4);
    h2d(dr, rec, l->bytes, b.fn);
    h2d(dq, q, (size_t) l->D * 4, b.fn);
    must(sjk_hip_record_scores(l, dr, dq, n, ds, nullptr), b.fn);
    d2h(scores, ds, (size_t) n * 4, b.fn);
}

void sj_kvarn_record_accum_v(const sj_kvarn_layout * l, const uint8_t * rec, const float * w, int n, float * acc) {
    if (n <= 0) return;
    CallBufs b("sj_kvarn_record_accum_v");
    uint8_t * dr = b.get<uint8_t>(l->bytes);
    float * dw = b.get<float>((size_t) l->G * 4);
    float * da = b.get<float>((size_t) l->D * 4);
    h2d(dr, rec, l->bytes, b.fn);
    h2d(dw, w, (size_t) n * 4, b.fn);
    h2d(da, acc, (size_t) l->D * 4, b.fn);
    must(sjk_hip_record_accum_v(l, dr, dw, n, da, nullptr), b.fn);
    d2h(acc, da, (size_t) l->D * 4, b.fn);
}

// ---------------------------------------------------------------------------------------------------
// journal policy, truncation, ring (sj_kvarn.h:1315-1407)
// ---------------------------------------------------------------------------------------------------

void sj_kvarn_policy_reset(sj_kvarn_policy * p) {
    p->B = p->B_prev = p->B_pending = p->sink;
    p->draining = 0;
}

void sj_kvarn_policy_init(sj_kvarn_policy * p, uint32_t sink, uint32_t tail, uint32_t tail_max, uint32_t group,
                          uint32_t flush_chunk) {
    p->sink = sink; p->tail = tail; p->tail_max = tail_max; p->group = group; p->flush_chunk = flush_chunk;
    sj_kvarn_policy_reset(p);
}

uint32_t sj_kvarn_group_floor(uint32_t sink, uint32_t group, uint32_t pos) {
    return pos <= sink ? pos : sink + group * ((pos - sink) / group);
}

uint32_t sj_kvarn_policy_begin_ubatch(sj_kvarn_policy * p, uint32_t pos0, uint32_t n_tokens) {
    const bool due = p->tail_max == 0 || p->draining || (pos0 > p->B && pos0 - p->B >= p->tail_max);
    p->B_pending = p->B;
    p->draining = 0;
    if (due && pos0 > p->sink + p->tail) {
        uint32_t target = sj_kvarn_group_floor(p->sink, p->group, pos0 - p->tail);
        if (target < p->B) target = p->B;
        if (p->tail_max > 0 && p->flush_chunk > 0 && n_tokens < p->group && target > p->B + p->group * p->flush_chunk) {
            target = p->B + p->group * p->flush_chunk;
            p->draining = 1;
        }
        p->B_pending = target;
    }
    return p->B_pending;
}

void sj_kvarn_policy_commit(sj_kvarn_policy * p) { p->B_prev = p->B; p->B = p->B_pending; }

uint32_t sj_kvarn_policy_idle(sj_kvarn_policy * p, uint32_t end, uint32_t keep_recent) {
    p->B_pending = p->B;
    if (p->tail_max == 0 || end <= p->sink + p->tail) return p->B;
    uint32_t target = sj_kvarn_group_floor(p->sink, p->group, end - p->tail);
    bool clamped = false;
    if (keep_recent > p->tail) {
        const uint32_t from = end > keep_recent ? end - keep_recent : 0;
        const uint32_t lim = from <= p->sink ? p->sink : sj_kvarn_group_floor(p->sink, p->group, from);
        if (lim < target) { target = lim; clamped = true; }
    }
    if (!clamped) p->draining = 0;
    if (target <= p->B) return p->B;
    p->B_pending = target;
    return target;
}

uint32_t sj_kvarn_policy_trunc_floor(const sj_kvarn_policy * p, uint32_t pos) {
    return (pos >= p->B || pos <= p->sink) ? pos : sj_kvarn_group_floor(p->sink, p->group, pos);
}

uint32_t sj_kvarn_policy_truncate(sj_kvarn_policy * p, uint32_t pos, uint32_t * n_dropped) {
    if (n_dropped) *n_dropped = 0;
    if (p->B_pending != p->B) return SJKVARN_NO_POS;
    const uint32_t r = sj_kvarn_policy_trunc_floor(p, pos);
    if (r < p->B) {
        const uint32_t nb = r > p->sink ? r : p->sink;
        if (n_dropped) *n_dropped = (p->B - nb) / p->group;
        p->B = p->B_prev = p->B_pending = nb;
        p->draining = 0;
    }
    return r;
}

uint32_t sj_kvarn_ring_capacity(uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t n_ubatch) {
    const uint32_t need = (tail > tail_max ? tail : tail_max) + group + 2u * n_ubatch;
    return (need + 127u) / 128u * 128u;
}

uint32_t sj_kvarn_ring_slot(uint32_t sink, uint32_t cap, uint32_t pos) { return (pos - sink) % cap; }

// ---------------------------------------------------------------------------------------------------
// per-layer cache on the device (sj_kvarn.h:1411-1603)
// ---------------------------------------------------------------------------------------------------

sj_kvarn_config sj_kvarn_config_default(int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch) {
    sj_kvarn_config c;
    c.head_dim = head_dim; c.n_head_kv = n_head_kv; c.group = SJKVARN_GROUP_DEFAULT; c.bits_k = 4; c.bits_v = 4;
    c.body = SJKVARN_BODY_AUTO; c.iters = SJKVARN_ITERS_DEFAULT; c.staging = SJKVARN_STAGING_TQ6_0;
    c.sink_type = SJKVARN_SINK_F16; c.sink = SJKVARN_SINK_DEFAULT; c.tail = SJKVARN_TAIL_DEFAULT;
    c.tail_max = SJKVARN_TAIL_MAX_DEFAULT; c.flush_chunk = 0; c.n_ubatch = n_ubatch; c.n_ctx = n_ctx;
    return c;
}

static size_t sink_entry_bytes(const sj_kvarn_layer * L) {
    return L->cfg.sink_type == SJKVARN_SINK_F16 ? (size_t) L->cfg.head_dim * 4 : 2 * L->stage_bytes;
}
static uint8_t * sink_entry(const sj_kvarn_layer * L, uint32_t pos, int h) {
    return L->sink + ((size_t) pos * (size_t) L->cfg.n_head_kv + (size_t) h) * sink_entry_bytes(L);
}
static uint8_t * ring_entry(const sj_kvarn_layer * L, uint32_t pos, int h) {
    return L->ring + ((size_t) sj_kvarn_ring_slot(L->cfg.sink, L->cap, pos) * (size_t) L->cfg.n_head_kv + (size_t) h) *
                         2 * L->stage_bytes;
}

uint8_t * sj_kvarn_layer_record(const sj_kvarn_layer * L, uint32_t g, int h) {
    const uint32_t blk = L->blocks ? L->blocks[g] : g;
    return L->body + ((size_t) blk * (size_t) L->cfg.n_head_kv + (size_t) h) * L->lay.bytes;
}

sjk_hip_view sjk_layer_view(const sj_kvarn_layer * L) {
    sjk_hip_view v;
    memset(&v, 0, sizeof(v));
    v.work = L->kstage;
    v.work_bytes = L->kstage ? sjk_hip_workspace_bytes(&L->lay, L->cfg.n_head_kv) : 0;
    v.lay = L->lay;
    v.n_head_kv = L->cfg.n_head_kv;
    v.staging = L->cfg.staging;
    v.sink_type = L->cfg.sink_type;
    v.S = L->cfg.sink;
    v.cap = L->cap;
    v.stage_bytes = L->stage_bytes;
    v.sink = L->sink;
    v.ring = L->ring;
    v.body = L->body;
    v.blocks = L->blocks ? (const uint32_t *) L->work : nullptr;
    return v;
}

void sj_kvarn_layer_free(sj_kvarn_layer * L) {
    if (L->vstage) rt_destroy(rt_of(L));
    if (L->ring) (void) hipFree(L->ring);
    if (L->sink) (void) hipFree(L->sink);
    if (L->owns_body && L->body) (void) hipFree(L->body);
    if (L->kstage) (void) hipFree(L->kstage);
    L->ring = L->sink = L->body = nullptr;
    L->blocks = nullptr;
    L->work = nullptr;
    L->owns_body = 0;
    L->kstage = L->vstage = nullptr;
}

// shared_ws: the workspace of the sequence's first layer (NULL: allocate the layer's own)
static int layer_setup(sj_kvarn_layer * L, const sj_kvarn_config * cfg, int own_body, uint16_t * shared_ws) {
    const int D = cfg->head_dim, H = cfg->n_head_kv;
    memset(L, 0, sizeof(*L));
    L->cfg = *cfg;
    L->cfg.body = sj_kvarn_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (D % SJKVARN_TQ6_QK || cfg->group % 16 || cfg->sink == 0 || cfg->sink % 64 || cfg->tail % (uint32_t) cfg->group ||
        (cfg->tail_max != 0 && (cfg->tail_max < cfg->tail || cfg->tail_max % 128)))
        return -10;
    const int rc = sj_kvarn_layout_init(&L->lay, D, cfg->group, cfg->bits_k, cfg->bits_v, L->cfg.body);
    if (rc) return rc;
    if (!sjk_hip_supported(&L->lay) || H <= 0) return SJK_ERR_UNSUPPORTED;
    L->cap = sj_kvarn_ring_capacity(cfg->tail, cfg->tail_max, (uint32_t) cfg->group, cfg->n_ubatch);
    L->n_groups = cfg->n_ctx > cfg->sink ? (cfg->n_ctx - cfg->sink + (uint32_t) cfg->group - 1) / (uint32_t) cfg->group : 1;
    L->stage_bytes = sj_kvarn_stage_row_bytes(cfg->staging, D);
    const size_t ring_b = (size_t) L->cap * H * 2 * L->stage_bytes;
    const size_t sink_b = (size_t) cfg->sink * H * sink_entry_bytes(L);
    const size_t body_b = (size_t) L->n_groups * H * L->lay.bytes;
    L->owns_body = own_body;
    if (hipMalloc((void **) &L->ring, ring_b) != hipSuccess || hipMalloc((void **) &L->sink, sink_b) != hipSuccess ||
        (own_body && hipMalloc((void **) &L->body, body_b) != hipSuccess)) {
        sj_kvarn_layer_free(L);
        return -11;
    }
    if (hipMemset(L->ring, 0, ring_b) != hipSuccess || hipMemset(L->sink, 0, sink_b) != hipSuccess ||
        (own_body && hipMemset(L->body, 0, body_b) != hipSuccess)) {
        sj_kvarn_layer_free(L);
        return -11;
    }
    if (!shared_ws && hipMalloc((void **) &L->kstage, sjk_hip_workspace_bytes(&L->lay, H)) != hipSuccess) {
        L->kstage = nullptr;
        sj_kvarn_layer_free(L);
        return -11;
    }
    if (shared_ws) L->kstage = shared_ws;    // set last: a failed set-up frees only what it allocated
    return 0;
}

int sj_kvarn_layer_init(sj_kvarn_layer * L, const sj_kvarn_config * cfg) {
    const int rc = layer_setup(L, cfg, 1, nullptr);
    if (rc) return rc;
    Rt * r = rt_create((size_t) L->n_groups + 3u);
    if (!r) { sj_kvarn_layer_free(L); return -11; }
    L->vstage = (uint16_t *) (void *) r;
    return 0;
}

// the host-array layer calls stage their rows in the layer's workspace (serialised with the layer's other use,
// as every call on a cache object is)
void sj_kvarn_layer_store(sj_kvarn_layer * L, uint32_t pos, const float * k_rot, const float * v_rot) {
    const size_t bytes = (size_t) L->cfg.n_head_kv * L->cfg.head_dim * 4;
    const sjk_hip_view v = sjk_layer_view(L);
    float * dk = (float *) sjk::ws_stage(v);
    float * dv = dk + (size_t) L->cfg.n_head_kv * L->cfg.head_dim;
    h2d(dk, k_rot, bytes, "sj_kvarn_layer_store");
    h2d(dv, v_rot, bytes, "sj_kvarn_layer_store");
    must(sjk_hip_layer_store(&v, pos, 1, dk, dv, 0, nullptr), "sj_kvarn_layer_store");
    null_sync("sj_kvarn_layer_store");
}

// seals on the layer's own stream after the work on the null stream (where a view's stores of an engine that
// does not pass streams go) and waits for that seal only
void sj_kvarn_layer_seal(sj_kvarn_layer * L, uint32_t B_from, uint32_t B_to) {
    const sjk_hip_view v = sjk_layer_view(L);
    Rt * r = rt_of(L);
    if (!r) {
        must(sjk_hip_commit(&v, 1, B_from, B_to, L->cfg.iters, nullptr), "sj_kvarn_layer_seal");
        null_sync("sj_kvarn_layer_seal");
        return;
    }
    must(rt_after_stores(r, r->st), "sj_kvarn_layer_seal");
    must(sjk_hip_commit(&v, 1, B_from, B_to, L->cfg.iters, r->st), "sj_kvarn_layer_seal");
    must(rt_wait(r, r->st), "sj_kvarn_layer_seal");
}

void sj_kvarn_layer_kv_row(const sj_kvarn_layer * L, uint32_t B, uint32_t pos, int h, float * k, float * v) {
    const size_t bytes = (size_t) L->cfg.head_dim * 4;
    const sjk_hip_view view = sjk_layer_view(L);
    float * dk = (float *) sjk::ws_stage(view);
    float * dv = dk + L->cfg.head_dim;
    must(sjk_hip_kv_rows(&view, B, pos, 1, h, dk, dv, nullptr), "sj_kvarn_layer_kv_row");
    d2h(k, dk, bytes, "sj_kvarn_layer_kv_row");
    d2h(v, dv, bytes, "sj_kvarn_layer_kv_row");
}

void sj_kvarn_layer_attend_row(const sj_kvarn_layer * L, uint32_t B, uint32_t N, const float * q_rot, int h, uint32_t qpos,
                               float scale, float * out_rot) {
    // one query row for KV head h: run the device attention with one query head per KV head and
    // the query placed at head h (the other heads get zero queries and are discarded)
    const int H = L->cfg.n_head_kv, D = L->cfg.head_dim;
    const size_t bytes = (size_t) H * D * 4;
    const sjk_hip_view v = sjk_layer_view(L);
    float * dq = (float *) sjk::ws_stage(v);
    float * dout = dq + (size_t) H * D;
    must_hip(hipMemset(dq, 0, bytes), "sj_kvarn_layer_attend_row");
    h2d(dq + (size_t) h * D, q_rot, (size_t) D * 4, "sj_kvarn_layer_attend_row");
    must(sjk_hip_attend(&v, B, N, qpos, 1, H, dq, scale, dout, nullptr), "sj_kvarn_layer_attend_row");
    d2h(out_rot, dout + (size_t) h * D, (size_t) D * 4, "sj_kvarn_layer_attend_row");
}

// The byte ranges a truncation clears in one layer (sj_kvarn.h:1581-1603): the records of groups [B_new, B_old)
// (in pool mode only the blocks the sequence holds), the sink entries of positions [resume, min(n_old, S)) and
// the ring rows of positions [max(resume, S), n_old) that can still be resident (the last cap of them), as
// contiguous runs.
static void truncate_runs(const sj_kvarn_layer * L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume,
                          std::vector<sjk::CopyRun> & runs) {
    const uint32_t S = L->cfg.sink, G = (uint32_t) L->cfg.group;
    const size_t H = (size_t) L->cfg.n_head_kv;
    auto add = [&](const uint8_t * p, size_t n) {
        if (!n) return;
        const uint64_t d = (uint64_t) (uintptr_t) p;
        if (!runs.empty() && runs.back().dst + runs.back().bytes == d) runs.back().bytes += n;
        else runs.push_back(sjk::CopyRun{0, d, n});
    };
    if (B_new < B_old)
        for (uint32_t g = (B_new - S) / G; g < (B_old - S) / G; ++g) {
            if (L->blocks && L->blocks[g] == SJKVARN_NO_BLOCK) continue;
            add(sj_kvarn_layer_record(L, g, 0), H * L->lay.bytes);
        }
    const uint32_t se = n_old < S ? n_old : S;
    if (resume < se) add(sink_entry(L, resume, 0), (size_t) (se - resume) * H * sink_entry_bytes(L));
    uint32_t from = resume > S ? resume : S;
    if (n_old > from && n_old - from > L->cap) from = n_old - L->cap;
    const size_t re = H * 2 * L->stage_bytes;
    while (from < n_old) {                                // slots of [from, n_old): one wrap of the ring at most
        const uint32_t slot = sj_kvarn_ring_slot(S, L->cap, from), room = L->cap - slot, left = n_old - from;
        const uint32_t k = left < room ? left : room;
        add(ring_entry(L, from, 0), (size_t) k * re);
        from += k;
    }
}

// Zero every run (synchronous, as the reference's memsets): one launch over the object's run table, which init
// sized for every run a truncation of the object can have; a table that does not fit (an object without a runtime)
// is cleared run by run. On the null stream, after the work enqueued there and on the object's store streams.
static int zero_runs(Rt * r, const std::vector<sjk::CopyRun> & runs) {
    if (runs.empty()) return 0;
    if (r) {
        const int rc = rt_after_stores(r, nullptr);
        if (rc) return rc;
    }
    if (r && runs.size() <= r->max_runs) {
        HIP_TRY(hipMemcpyAsync(r->d_runs, runs.data(), runs.size() * sizeof(sjk::CopyRun), hipMemcpyHostToDevice, nullptr));
        if (sjk::sjk_zero_runs(r->d_runs, (int) runs.size(), nullptr)) return hip_fail(hipGetLastError(), "truncate scrub");
    } else {
        for (const sjk::CopyRun & c : runs) HIP_TRY(hipMemsetAsync((void *) (uintptr_t) c.dst, 0, c.bytes, nullptr));
    }
    HIP_TRY(hipStreamSynchronize(nullptr));
    if (r) { r->n_store = 0; r->store_many = false; }
    return 0;
}

void sj_kvarn_layer_truncate(sj_kvarn_layer * L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume) {
    std::vector<sjk::CopyRun> runs;
    truncate_runs(L, B_old, B_new, n_old, resume, runs);
    must(zero_runs(rt_of(L), runs), "sj_kvarn_layer_truncate");
}

const char * sj_kvarn_strerror(int code) {
    switch (code) {
    case 0: return "ok";
    case -1: return "layout: head_dim must be a power of two >= 32 and group a multiple of 16";
    case -2: return "layout: bits_k and bits_v must be 2, 3 or 4";
    case -3: return "layout: unknown body type";
    case -4: return "layout: trellis bodies need 3/3, 3/2 or 2/2 bits, group 128 and head_dim a multiple of 128";
    case -10: return "config: head_dim % 128, group % 16, sink (non-zero, % 64), tail % group or tail_max invalid";
    case -11: return "out of memory";
    case SJKVARN_ERR_ARG: return "invalid argument";
    case SJKVARN_ERR_NOMEM: return "out of memory";
    case SJKVARN_ERR_BUFFER: return "destination buffer too small for the sequence state";
    case SJKVARN_ERR_TRUNCATED: return "state stream is shorter than its header says";
    case SJKVARN_ERR_MAGIC: return "not an SJ-KVaRN sequence state (bad magic)";
    case SJKVARN_ERR_VERSION: return "unsupported SJ-KVaRN state version";
    case SJKVARN_ERR_FORMAT: return "state was written with a different record/staging byte format";
    case SJKVARN_ERR_CORRUPT: return "state checksum or consistency check failed";
    case SJKVARN_ERR_PENDING: return "a seal is pending (call commit first)";
    case SJKVARN_ERR_CAPACITY: return "state does not fit this cache (context, ring or group capacity)";
    case SJKVARN_ERR_POOL_FULL: return "record pool has no free block";
    case SJKVARN_ERR_HEAD_DIM: return "config mismatch: head_dim";
    case SJKVARN_ERR_N_HEAD_KV: return "config mismatch: n_head_kv";
    case SJKVARN_ERR_GROUP: return "config mismatch: group size";
    case SJKVARN_ERR_SINK: return "config mismatch: sink length or sink type";
    case SJKVARN_ERR_BITS: return "config mismatch: bits_k/bits_v";
    case SJKVARN_ERR_BODY: return "config mismatch: body type (scalar/trellis)";
    case SJKVARN_ERR_ITERS: return "config mismatch: variance-balancing iterations";
    case SJKVARN_ERR_STAGING: return "config mismatch: staging type";
    case SJKVARN_ERR_TAIL: return "config mismatch: tail, tail_max or flush_chunk";
    case SJKVARN_ERR_ROTATION: return "config mismatch: rotation";
    case SJKVARN_ERR_CODEBOOK: return "config mismatch: trellis codebook";
    case SJKVARN_ERR_N_LAYERS: return "config mismatch: number of layers";
    case SJK_ERR_DEVICE: return "HIP runtime error (see sjk_last_error)";
    case SJK_ERR_UNSUPPORTED: return "shape not supported by the HIP kernels (head_dim 128/256, group 128)";
    default: return "unknown SJ-KVaRN status code";
    }
}

// ---------------------------------------------------------------------------------------------------
// paged pool / sequence (sj_kvarn.h:1645-1809)
// ---------------------------------------------------------------------------------------------------

int sj_kvarn_pool_init(sj_kvarn_pool * pool, const sj_kvarn_config * cfg, int n_layers, uint32_t n_blocks) {
    memset(pool, 0, sizeof(*pool));
    if (n_layers <= 0 || n_blocks == 0 || cfg->n_head_kv <= 0) return SJKVARN_ERR_ARG;
    pool->cfg = *cfg;
    pool->cfg.body = sj_kvarn_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    const int rc = sj_kvarn_layout_init(&pool->lay, cfg->head_dim, cfg->group, cfg->bits_k, cfg->bits_v, pool->cfg.body);
    if (rc) return rc;
    pool->n_layers = n_layers;
    pool->n_blocks = n_blocks;
    const size_t body_b = (size_t) n_layers * n_blocks * (size_t) cfg->n_head_kv * pool->lay.bytes;
    pool->free_ids = (uint32_t *) malloc((size_t) n_blocks * sizeof(uint32_t));
    if (!pool->free_ids || hipMalloc((void **) &pool->body, body_b) != hipSuccess ||
        hipMemset(pool->body, 0, body_b) != hipSuccess) {
        sj_kvarn_pool_free(pool);
        return SJKVARN_ERR_NOMEM;
    }
    for (uint32_t i = 0; i < n_blocks; ++i) pool->free_ids[i] = n_blocks - 1u - i;  // LIFO: block 0 first
    pool->n_free = n_blocks;
    return 0;
}

void sj_kvarn_pool_free(sj_kvarn_pool * pool) {
    if (pool->body) (void) hipFree(pool->body);
    free(pool->free_ids);
    pool->body = nullptr;
    pool->free_ids = nullptr;
    pool->n_free = 0;
}

uint32_t sj_kvarn_pool_alloc(sj_kvarn_pool * pool) { return pool->n_free ? pool->free_ids[--pool->n_free] : SJKVARN_NO_BLOCK; }

void sj_kvarn_pool_release(sj_kvarn_pool * pool, uint32_t id) {
    if (id != SJKVARN_NO_BLOCK && pool->n_free < pool->n_blocks) pool->free_ids[pool->n_free++] = id;
}

// the device copy of a sequence's block table lives in layers[0].work (shared by every layer): entries [g0, g1)
// written on stream st from the kernel arguments (the host table may change as soon as this returns); wait: the
// host waits for st
static int seq_sync_blocks(sj_kvarn_seq * s, uint32_t g0 = 0, uint32_t g1 = UINT32_MAX, hipStream_t st = nullptr,
                           bool wait = true) {
    if (!s->pool) return 0;
    if (g1 > s->layers[0].n_groups) g1 = s->layers[0].n_groups;
    if (g0 >= g1) return 0;
    if (sjk::sjk_set_words((uint32_t *) s->layers[0].work + g0, s->blocks + g0, g1 - g0, st))
        return hip_fail(hipGetLastError(), "block table");
    if (wait) HIP_TRY(hipStreamSynchronize(st));
    return 0;
}

int sj_kvarn_seq_init(sj_kvarn_seq * s, const sj_kvarn_config * cfg, int n_layers, sj_kvarn_pool * pool) {
    memset(s, 0, sizeof(*s));
    if (n_layers <= 0) return SJKVARN_ERR_ARG;
    s->cfg = *cfg;
    s->cfg.body = sj_kvarn_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (pool) {
        const sj_kvarn_config * pc = &pool->cfg;
        if (pool->n_layers != n_layers || pc->head_dim != cfg->head_dim || pc->n_head_kv != cfg->n_head_kv ||
            pc->group != cfg->group || pc->bits_k != cfg->bits_k || pc->bits_v != cfg->bits_v || pc->body != s->cfg.body)
            return SJKVARN_ERR_ARG;
    }
    s->n_layers = n_layers;
    s->pool = pool;
    s->layers = (sj_kvarn_layer *) calloc((size_t) n_layers, sizeof(sj_kvarn_layer));
    if (!s->layers) return SJKVARN_ERR_NOMEM;
    // one attention workspace for the sequence (its layers are used one at a time, like the sequence)
    for (int il = 0; il < n_layers; ++il) {
        const int rc = layer_setup(&s->layers[il], cfg, pool == nullptr, il ? s->layers[0].kstage : nullptr);
        if (rc) { s->n_layers = il; sj_kvarn_seq_free(s); return rc; }
    }
    if (pool) {
        const uint32_t ng = s->layers[0].n_groups;
        s->blocks = (uint32_t *) malloc((size_t) ng * sizeof(uint32_t));
        void * d_blocks = nullptr;
        if (!s->blocks || hipMalloc(&d_blocks, (size_t) ng * 4) != hipSuccess) { sj_kvarn_seq_free(s); return SJKVARN_ERR_NOMEM; }
        for (uint32_t g = 0; g < ng; ++g) s->blocks[g] = SJKVARN_NO_BLOCK;
        for (int il = 0; il < n_layers; ++il) {
            s->layers[il].body = pool->body + (size_t) il * pool->n_blocks * (size_t) cfg->n_head_kv * pool->lay.bytes;
            s->layers[il].blocks = s->blocks;
            s->layers[il].work = d_blocks;
        }
        if (seq_sync_blocks(s)) { sj_kvarn_seq_free(s); return SJK_ERR_DEVICE; }
    }
    Rt * r = rt_create((size_t) n_layers * ((size_t) s->layers[0].n_groups + 3u));
    if (!r) { sj_kvarn_seq_free(s); return SJKVARN_ERR_NOMEM; }
    s->layers[0].vstage = (uint16_t *) (void *) r;
    sj_kvarn_policy_init(&s->pol, cfg->sink, cfg->tail, cfg->tail_max, (uint32_t) cfg->group, cfg->flush_chunk);
    s->n = 0;
    return 0;
}

static int seq_release(sj_kvarn_seq * s, uint32_t g0, uint32_t g1) {
    if (!s->pool || !s->blocks) return 0;
    for (uint32_t g = g0; g < g1 && g < s->layers[0].n_groups; ++g) {
        sj_kvarn_pool_release(s->pool, s->blocks[g]);
        s->blocks[g] = SJKVARN_NO_BLOCK;
    }
    return seq_sync_blocks(s, g0, g1);
}

// take pool blocks for groups [g0, g1) on the host; the caller copies the table's range to the device
static int seq_reserve(sj_kvarn_seq * s, uint32_t g0, uint32_t g1) {
    if (!s->pool) return 0;
    if (g1 > s->layers[0].n_groups) return SJKVARN_ERR_CAPACITY;
    for (uint32_t g = g0; g < g1; ++g) {
        if (s->blocks[g] != SJKVARN_NO_BLOCK) continue;
        s->blocks[g] = sj_kvarn_pool_alloc(s->pool);
        if (s->blocks[g] == SJKVARN_NO_BLOCK) {
            while (g-- > g0) { sj_kvarn_pool_release(s->pool, s->blocks[g]); s->blocks[g] = SJKVARN_NO_BLOCK; }
            return SJKVARN_ERR_POOL_FULL;
        }
    }
    return 0;
}

// (an asynchronous state job in flight is waited for when the runtime of layer 0 goes, and not applied)
void sj_kvarn_seq_free(sj_kvarn_seq * s) {
    if (s->layers) {
        if (s->pool && s->blocks && s->n_layers > 0) {
            for (uint32_t g = 0; g < s->layers[0].n_groups; ++g) sj_kvarn_pool_release(s->pool, s->blocks[g]);
            if (s->layers[0].work) (void) hipFree(s->layers[0].work);
        }
        for (int il = 1; il < s->n_layers; ++il) s->layers[il].kstage = nullptr;   // layer 0 owns the workspace
        for (int il = 0; il < s->n_layers; ++il) sj_kvarn_layer_free(&s->layers[il]);
    }
    free(s->layers);
    free(s->blocks);
    s->layers = nullptr;
    s->blocks = nullptr;
    s->n_layers = 0;
    s->n = 0;
}

// the truncation scrub of every layer of a sequence in one launch
static int seq_scrub(sj_kvarn_seq * s, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume) {
    std::vector<sjk::CopyRun> runs;
    for (int il = 0; il < s->n_layers; ++il) truncate_runs(&s->layers[il], B_old, B_new, n_old, resume, runs);
    return zero_runs(rt_of(s), runs);
}

static int seq_reset_rc(sj_kvarn_seq * s) {
    int rc = seq_scrub(s, s->pol.B, s->cfg.sink, s->n, 0);
    if (!rc) rc = seq_release(s, 0, s->layers[0].n_groups);
    if (rc) return rc;
    sj_kvarn_policy_reset(&s->pol);
    s->n = 0;
    return 0;
}

void sj_kvarn_seq_reset(sj_kvarn_seq * s) { must(seq_reset_rc(s), "sj_kvarn_seq_reset"); }

// Seal [B, B_pending) in every layer with one launch (64 layers a launch), then commit; a failure leaves the
// policy as it was. host_wait: the drop-in calls seal on the sequence's own stream after its stores and wait for
// that seal only; otherwise the seal is enqueued on `st`, after what the caller enqueued there before, and the call
// returns without waiting (work the caller enqueues on st afterwards sees the records).
static int seq_seal_commit(sj_kvarn_seq * s, const sj_kvarn_policy * before, bool host_wait, hipStream_t st) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group;
    if (s->pol.B_pending > s->pol.B) {
        Rt * r = rt_of(s);
        if (host_wait && r) {
            st = r->st;
            const int rc = rt_after_stores(r, st);
            if (rc) { s->pol = *before; return rc; }
        }
        const uint32_t g0 = (s->pol.B - S) / G, g1 = (s->pol.B_pending - S) / G;
        int rc = seq_reserve(s, g0, g1);
        if (!rc) rc = seq_sync_blocks(s, g0, g1, st, false);
        if (rc) { s->pol = *before; return rc; }
        sjk_hip_view views[64];
        for (int il = 0; il < s->n_layers; il += 64) {
            const int nl = s->n_layers - il < 64 ? s->n_layers - il : 64;
            for (int k = 0; k < nl; ++k) views[k] = sjk_layer_view(&s->layers[il + k]);
            rc = sjk_hip_commit(views, nl, s->pol.B, s->pol.B_pending, s->cfg.iters, st);
            if (rc) { s->pol = *before; return rc; }
        }
        if (host_wait) {
            rc = r ? rt_wait(r, st) : (hipStreamSynchronize(st) == hipSuccess ? 0 : SJK_ERR_DEVICE);
            if (rc) { s->pol = *before; return rc; }
        } else {
            rt_note_store(r, st);     // the sequence's later scrubs and state transfers wait for this seal too
        }
    }
    sj_kvarn_policy_commit(&s->pol);
    return 0;
}

int sj_kvarn_seq_begin_ubatch(sj_kvarn_seq * s, uint32_t pos0, uint32_t n_tokens) {
    const sj_kvarn_policy before = s->pol;
    if (pos0 > s->n) return SJKVARN_ERR_ARG;
    sj_kvarn_policy_begin_ubatch(&s->pol, pos0, n_tokens);
    return seq_seal_commit(s, &before, true, nullptr);
}

int sjk_hip_seq_begin_ubatch(sj_kvarn_seq * s, uint32_t pos0, uint32_t n_tokens, void * stream) {
    const sj_kvarn_policy before = s->pol;
    if (pos0 > s->n) return SJKVARN_ERR_ARG;
    sj_kvarn_policy_begin_ubatch(&s->pol, pos0, n_tokens);
    return seq_seal_commit(s, &before, false, (hipStream_t) stream);
}

void sj_kvarn_seq_store(sj_kvarn_seq * s, uint32_t pos, const float * k_rot, const float * v_rot) {
    const size_t stride = (size_t) s->cfg.n_head_kv * (size_t) s->cfg.head_dim;
    for (int il = 0; il < s->n_layers; ++il)
        sj_kvarn_layer_store(&s->layers[il], pos, k_rot + il * stride, v_rot + il * stride);
    if (pos + 1u > s->n) s->n = pos + 1u;
}

int sj_kvarn_seq_idle(sj_kvarn_seq * s, uint32_t keep_recent) {
    const sj_kvarn_policy before = s->pol;
    sj_kvarn_policy_idle(&s->pol, s->n, keep_recent);
    return seq_seal_commit(s, &before, true, nullptr);
}

int sjk_hip_seq_idle(sj_kvarn_seq * s, uint32_t keep_recent, void * stream) {
    const sj_kvarn_policy before = s->pol;
    sj_kvarn_policy_idle(&s->pol, s->n, keep_recent);
    return seq_seal_commit(s, &before, false, (hipStream_t) stream);
}

uint32_t sj_kvarn_seq_truncate(sj_kvarn_seq * s, uint32_t pos) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group, B_old = s->pol.B, n_old = s->n;
    const uint32_t r = sj_kvarn_policy_truncate(&s->pol, pos, nullptr);
    if (r == SJKVARN_NO_POS) return r;
    must(seq_scrub(s, B_old, s->pol.B, n_old, r), "sj_kvarn_seq_truncate");
    if (s->pol.B < B_old) must(seq_release(s, (s->pol.B - S) / G, (B_old - S) / G), "sj_kvarn_seq_truncate");
    if (r < s->n) s->n = r;
    return r;
}

void sj_kvarn_seq_attend_row(const sj_kvarn_seq * s, int il, const float * q_rot, int h, uint32_t qpos, float scale,
                             float * out_rot) {
    sj_kvarn_layer_attend_row(&s->layers[il], s->pol.B, s->n, q_rot, h, qpos, scale, out_rot);
}

// device twins of seq_store / seq_attend_row, one layer per call (an engine stores and attends layer by
// layer): a store of [pos0, pos0 + n_pos) into any layer extends the sequence's position count, which
// the attention of every layer then covers, as after the reference's all-layer store of a position
// (sj_kvarn.h:1779-1792, 1806-1809)
int sjk_hip_seq_store(sj_kvarn_seq * s, int il, uint32_t pos0, uint32_t n_pos, const float * d_k, const float * d_v,
                      int rotate, void * stream) {
    if (il < 0 || il >= s->n_layers || pos0 > s->n) return SJKVARN_ERR_ARG;
    const sjk_hip_view v = sjk_layer_view(&s->layers[il]);
    const int rc = sjk_hip_layer_store(&v, pos0, n_pos, d_k, d_v, rotate, stream);
    if (rc == 0 && pos0 + n_pos > s->n) s->n = pos0 + n_pos;
    if (rc == 0) rt_note_store(rt_of(s), (hipStream_t) stream);
    return rc;
}

int sjk_hip_seq_attend(const sj_kvarn_seq * s, int il, uint32_t qpos0, int n_q, int n_head, const float * d_q,
                       float scale, float * d_out, void * stream) {
    if (il < 0 || il >= s->n_layers) return SJKVARN_ERR_ARG;
    const sjk_hip_view v = sjk_layer_view(&s->layers[il]);
    return sjk_hip_attend(&v, s->pol.B, s->n, qpos0, n_q, n_head, d_q, scale, d_out, stream);
}

// layer il of a decode batch of sequences, in as few launches as the kernels take
int sjk_hip_seq_store_batch(const sjk_hip_seq_job * jobs, int n_jobs, int il, uint32_t n_pos, int rotate, void * stream) {
    sjk_hip_store_job sj[16];
    for (int k0 = 0; k0 < n_jobs; k0 += 16) {
        const int n = n_jobs - k0 < 16 ? n_jobs - k0 : 16;
        for (int k = 0; k < n; ++k) {
            const sjk_hip_seq_job & J = jobs[k0 + k];
            if (!J.seq || il < 0 || il >= J.seq->n_layers || J.pos0 > J.seq->n) return SJKVARN_ERR_ARG;
            sj[k].v = sjk_layer_view(&J.seq->layers[il]);
            sj[k].pos0 = J.pos0; sj[k].d_k = J.d_k; sj[k].d_v = J.d_v;
        }
        const int rc = sjk_hip_store_batch(sj, n, n_pos, rotate, stream);
        if (rc) return rc;
        for (int k = 0; k < n; ++k) {
            sj_kvarn_seq * s = jobs[k0 + k].seq;
            if (jobs[k0 + k].pos0 + n_pos > s->n) s->n = jobs[k0 + k].pos0 + n_pos;
            rt_note_store(rt_of(s), (hipStream_t) stream);
        }
    }
    return 0;
}

int sjk_hip_seq_attend_batch(const sjk_hip_seq_job * jobs, int n_jobs, int il, int n_q, int n_head, float scale,
                             void * stream) {
    sjk_hip_attend_job aj[8];
    for (int k0 = 0; k0 < n_jobs; k0 += 8) {
        const int n = n_jobs - k0 < 8 ? n_jobs - k0 : 8;
        for (int k = 0; k < n; ++k) {
            const sjk_hip_seq_job & J = jobs[k0 + k];
            if (!J.seq || il < 0 || il >= J.seq->n_layers) return SJKVARN_ERR_ARG;
            aj[k].v = sjk_layer_view(&J.seq->layers[il]);
            aj[k].B = J.seq->pol.B; aj[k].N = J.seq->n; aj[k].qpos0 = J.pos0;
            aj[k].d_q = J.d_q; aj[k].d_out = J.d_out;
        }
        const int rc = sjk_hip_attend_batch(aj, n, n_q, n_head, scale, stream);
        if (rc) return rc;
    }
    return 0;
}

// ---------------------------------------------------------------------------------------------------
// sequence state stream (sj_kvarn.h:1811-2034): byte layout of the reference; the device pieces are
// gathered / scattered on the device and cross to the host in 64 MB chunks
// ---------------------------------------------------------------------------------------------------

static void le32(uint8_t * p, uint32_t v) { p[0] = (uint8_t) v; p[1] = (uint8_t) (v >> 8); p[2] = (uint8_t) (v >> 16); p[3] = (uint8_t) (v >> 24); }
static void le64(uint8_t * p, uint64_t v) { le32(p, (uint32_t) v); le32(p + 4, (uint32_t) (v >> 32)); }
static uint32_t rd32(const uint8_t * p) { return (uint32_t) p[0] | (uint32_t) p[1] << 8 | (uint32_t) p[2] << 16 | (uint32_t) p[3] << 24; }
static uint64_t rd64(const uint8_t * p) { return (uint64_t) rd32(p) | (uint64_t) rd32(p + 4) << 32; }

static uint64_t codebook_id(int body, int bits_k, int bits_v) {
    if (body != SJKVARN_BODY_TRELLIS) return 0;
    static const uint16_t cb3k[] = SJK_CB3_K_INIT, cb3v[] = SJK_CB3_V_INIT, cb2k[] = SJK_CB2_K_INIT, cb2v[] = SJK_CB2_V_INIT;
    uint64_t h = FNV0;
    h = bits_k == 3 ? fnv1a(cb3k, sizeof(cb3k), h) : fnv1a(cb2k, sizeof(cb2k), h);
    h = bits_v == 3 ? fnv1a(cb3v, sizeof(cb3v), h) : fnv1a(cb2v, sizeof(cb2v), h);
    return h;
}

static size_t layer_payload(const sj_kvarn_config * c, const sj_kvarn_layout * lay, uint32_t n, uint32_t B) {
    const size_t H = (size_t) c->n_head_kv, rr = 2 * sj_kvarn_stage_row_bytes(c->staging, c->head_dim);
    const size_t sr = c->sink_type == SJKVARN_SINK_F16 ? (size_t) c->head_dim * 4 : rr;
    const uint32_t ns = n < c->sink ? n : c->sink, nr = (B - c->sink) / (uint32_t) c->group, nt = n > B ? n - B : 0;
    return (size_t) ns * H * sr + (size_t) nr * H * lay->bytes + (size_t) nt * H * rr;
}

size_t sj_kvarn_seq_state_size(const sj_kvarn_seq * s) {
    return SJKVARN_STATE_HEADER_BYTES + (size_t) s->n_layers * layer_payload(&s->cfg, &s->layers[0].lay, s->n, s->pol.B) + 8;
}

size_t sj_kvarn_state_size_max(const sj_kvarn_config * cfg, int n_layers) {
    sj_kvarn_config c = *cfg;
    sj_kvarn_layout lay;
    c.body = sj_kvarn_body_resolve(cfg->body, cfg->bits_k, cfg->bits_v);
    if (n_layers <= 0 || sj_kvarn_layout_init(&lay, c.head_dim, c.group, c.bits_k, c.bits_v, c.body)) return 0;
    const uint32_t G = (uint32_t) c.group;
    const uint32_t B_all = c.n_ctx > c.sink ? c.sink + G * ((c.n_ctx - c.sink + G - 1u) / G) : c.sink;
    const size_t a = layer_payload(&c, &lay, c.n_ctx, c.sink), b = layer_payload(&c, &lay, c.n_ctx, B_all);
    return SJKVARN_STATE_HEADER_BYTES + (size_t) n_layers * (a > b ? a : b) + 8;
}

static const uint8_t k_state_magic[8] = {'S', 'J', 'K', 'V', 'S', 'E', 'Q', 0};

}  // extern "C"

namespace {

// The device pieces of a state stream (sink, records, ring rows of every layer, in stream order) move in
// chunks through the object's two device stages and two pinned host buffers, on its own stream: writing, chunk
// k is gathered on the device (one sjk_copy_runs launch) and copied to pinned memory while the host copies chunk
// k - 1 into the caller's buffer and extends the stream's FNV-1a checksum over it; reading, the host fills the
// pinned buffer of chunk k while the device copies in and scatters chunk k - 1. Contiguous pieces merge into one
// run. The buffers are the object's (allocated by its first state call, before the sequence is touched).
constexpr size_t XFER_STAGE = (size_t) 32 << 20;   // stream bytes per chunk
constexpr size_t XFER_RUNS = 1 << 15;              // runs per chunk

int rt_xfer_buffers(Rt * r) {
    if (r->xfer_ready) return 0;
    for (int b = 0; b < 2; ++b) {
        if (!r->dstage[b]) HIP_TRY(hipMalloc((void **) &r->dstage[b], XFER_STAGE));
        if (!r->druns[b]) HIP_TRY(hipMalloc((void **) &r->druns[b], XFER_RUNS * sizeof(sjk::CopyRun)));
        if (!r->hpin[b]) HIP_TRY(hipHostMalloc((void **) &r->hpin[b], XFER_STAGE, hipHostMallocDefault));
        if (!r->hruns[b]) HIP_TRY(hipHostMalloc((void **) &r->hruns[b], XFER_RUNS * sizeof(sjk::CopyRun), hipHostMallocDefault));
        if (!r->xev[b]) HIP_TRY(hipEventCreateWithFlags(&r->xev[b], hipEventDisableTiming));
    }
    r->xfer_ready = true;
    return 0;
}

struct Xfer {
    bool out;                            // device -> host stream (state write)
    uint8_t * host;                      // stream byte of the next chunk's first byte
    uint64_t fnv = 0;                    // write: checksum of the stream bytes handed to the host so far
    Rt * r = nullptr;
    hipStream_t st = nullptr;
    bool busy[2] = {};                   // chunk in flight in buffer b
    uint8_t * dest[2] = {};              // write: where chunk b goes in the caller's buffer
    size_t len[2] = {};
    int cur = 0;                         // buffer of the chunk being assembled
    size_t fill = 0, n_runs = 0;

    Xfer(bool o, uint8_t * h, uint64_t f) : out(o), host(h), fnv(f) {}
    Xfer(const Xfer &) = delete;
    Xfer & operator=(const Xfer &) = delete;

    // the object's buffers; its stream, ordered after the work enqueued on the null stream and its store streams
    int open(Rt * rt) {
        r = rt;
        int rc = rt_xfer_buffers(r);
        if (!rc) rc = rt_after_stores(r, r->st);
        st = r->st;
        return rc;
    }

    ~Xfer() {
        if (st) (void) hipStreamSynchronize(st);
    }

    // wait for the chunk in buffer b; writing, hand its bytes to the caller and the checksum
    int retire(int b) {
        if (!busy[b]) return 0;
        HIP_TRY(hipEventSynchronize(r->xev[b]));
        if (out) {
            memcpy(dest[b], r->hpin[b], len[b]);
            fnv = fnv1a(dest[b], len[b], fnv);
        }
        busy[b] = false;
        return 0;
    }

    int region(const uint8_t * dev, size_t bytes) {
        while (bytes) {
            const size_t take = bytes < XFER_STAGE - fill ? bytes : XFER_STAGE - fill;
            const uint64_t d = (uint64_t) (uintptr_t) dev, sg = (uint64_t) (uintptr_t) (r->dstage[cur] + fill);
            const sjk::CopyRun run = out ? sjk::CopyRun{d, sg, take} : sjk::CopyRun{sg, d, take};
            sjk::CopyRun * rs = r->hruns[cur];
            if (n_runs && rs[n_runs - 1].src + rs[n_runs - 1].bytes == run.src && rs[n_runs - 1].dst + rs[n_runs - 1].bytes == run.dst)
                rs[n_runs - 1].bytes += take;
            else
                rs[n_runs++] = run;
            fill += take; dev += take; bytes -= take;
            if (fill == XFER_STAGE || n_runs == XFER_RUNS) {
                const int rc = flush();
                if (rc) return rc;
            }
        }
        return 0;
    }

    // submit the chunk being assembled, then finish the one before it (which overlaps this one)
    int flush() {
        if (!fill) return 0;
        const int b = cur;
        if (!out) {
            memcpy(r->hpin[b], host, fill);
            HIP_TRY(hipMemcpyAsync(r->dstage[b], r->hpin[b], fill, hipMemcpyHostToDevice, st));
        }
        HIP_TRY(hipMemcpyAsync(r->druns[b], r->hruns[b], n_runs * sizeof(sjk::CopyRun), hipMemcpyHostToDevice, st));
        if (sjk::sjk_copy_runs(r->druns[b], (int) n_runs, st)) return hip_fail(hipGetLastError(), "sjk_copy_runs");
        if (out) HIP_TRY(hipMemcpyAsync(r->hpin[b], r->dstage[b], fill, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipEventRecord(r->xev[b], st));
        busy[b] = true;
        dest[b] = host;
        len[b] = fill;
        host += fill;
        fill = 0;
        n_runs = 0;
        cur ^= 1;
        // the other buffer's chunk (submitted before this one) is done next; the buffer the next chunk assembles
        // in is then free: its host side (pinned bytes, run table) was last read by that earlier chunk
        return retire(cur);
    }

    int finish() {
        int rc = flush();
        if (!rc) rc = retire(cur ^ 1);
        if (!rc) rc = retire(cur);
        if (!rc) HIP_TRY(hipStreamSynchronize(st));
        return rc;
    }
};

// the pieces of one layer in stream order: sink rows [0, min(n, S)), records of [S, B), ring rows [B, n); emit(p, n)
// gets each piece's device address and length
template <typename F>
int layer_pieces(const sj_kvarn_layer * L, uint32_t n, uint32_t B, F && emit) {
    const uint32_t S = L->cfg.sink, G = (uint32_t) L->cfg.group;
    const int H = L->cfg.n_head_kv;
    const uint32_t ns = n < S ? n : S;
    int rc = emit(L->sink, (size_t) ns * H * sink_entry_bytes(L));
    const uint32_t n_rec = (B - S) / G;
    const size_t gb = (size_t) H * L->lay.bytes;
    for (uint32_t g = 0; g < n_rec && !rc; ++g) rc = emit(sj_kvarn_layer_record(L, g, 0), gb);
    const size_t re = (size_t) H * 2 * L->stage_bytes;
    for (uint32_t pos = B; pos < n && !rc; ++pos) rc = emit(ring_entry(L, pos, 0), re);
    return rc;
}

int xfer_layer(Xfer & x, const sj_kvarn_layer * L, uint32_t n, uint32_t B) {
    return layer_pieces(L, n, B, [&](const uint8_t * p, size_t b) { return x.region(p, b); });
}

// the runs between a sequence's pieces and a contiguous device image of the stream payload (gather: pieces ->
// image; scatter: image -> pieces), contiguous runs merged
std::vector<sjk::CopyRun> image_runs(const sj_kvarn_seq * s, uint32_t n, uint32_t B, uint8_t * image, bool gather) {
    std::vector<sjk::CopyRun> runs;
    size_t off = 0;
    for (int il = 0; il < s->n_layers; ++il)
        layer_pieces(&s->layers[il], n, B, [&](const uint8_t * p, size_t b) {
            if (!b) return 0;
            const uint64_t d = (uint64_t) (uintptr_t) p, im = (uint64_t) (uintptr_t) (image + off);
            const sjk::CopyRun run = gather ? sjk::CopyRun{d, im, b} : sjk::CopyRun{im, d, b};
            if (!runs.empty() && runs.back().src + runs.back().bytes == run.src && runs.back().dst + runs.back().bytes == run.dst)
                runs.back().bytes += b;
            else
                runs.push_back(run);
            off += b;
            return 0;
        });
    return runs;
}

// one copy_runs launch over the runs (through the object's run table) on its stream, waited for on the host
int run_copy(Rt * r, const std::vector<sjk::CopyRun> & runs) {
    if (runs.empty()) return 0;
    if (runs.size() > r->max_runs) { sjk::set_error("state image: more runs than the run table holds"); return SJK_ERR_DEVICE; }
    HIP_TRY(hipMemcpyAsync(r->d_runs, runs.data(), runs.size() * sizeof(sjk::CopyRun), hipMemcpyHostToDevice, r->st));
    if (sjk::sjk_copy_runs(r->d_runs, (int) runs.size(), r->st)) return hip_fail(hipGetLastError(), "sjk_copy_runs");
    return rt_wait(r, r->st);
}

int rt_snapshot(Rt * r, size_t bytes) {
    if (r->snap_cap >= bytes) return 0;
    if (r->snap) (void) hipFree(r->snap);
    r->snap = nullptr;
    r->snap_cap = 0;
    HIP_TRY(hipMalloc((void **) &r->snap, bytes ? bytes : 1));
    r->snap_cap = bytes;
    return 0;
}

// An asynchronous state save or restore: a host thread moves the stream payload between the object's device
// snapshot and the caller's buffer through the pinned buffers, on the object's transfer stream.
struct StateJob {
    bool out;                         // save (snapshot -> dst)
    uint8_t * host;                   // save: the caller's buffer; restore: the stream
    size_t total = 0;                 // stream bytes (header + payload + checksum)
    uint64_t fnv = 0;                 // save: checksum of the header
    uint32_t n = 0, B = 0, B_prev = 0, draining = 0;   // restore: the header's policy state
    std::thread th;
    std::mutex mu;
    bool done = false;
    int status = 0;
    char err[256] = "";
};

int job_run(Rt * r, StateJob * j) {
    const size_t payload = j->total - SJKVARN_STATE_HEADER_BYTES - 8;
    uint8_t * h = j->host + SJKVARN_STATE_HEADER_BYTES;
    if (!j->out && fnv1a(j->host, j->total - 8, FNV0) != rd64(j->host + j->total - 8)) return SJKVARN_ERR_CORRUPT;
    size_t len[2] = {};
    uint8_t * where[2] = {};
    bool busy[2] = {};
    uint64_t fnv = j->fnv;
    int b = 0;
    for (size_t off = 0; off < payload || busy[0] || busy[1]; b ^= 1) {
        if (busy[b]) {                                      // the chunk submitted two steps ago
            HIP_TRY(hipEventSynchronize(r->xev[b]));
            if (j->out) {
                memcpy(where[b], r->hpin[b], len[b]);
                fnv = fnv1a(where[b], len[b], fnv);
            }
            busy[b] = false;
        }
        if (off < payload) {
            const size_t take = payload - off < XFER_STAGE ? payload - off : XFER_STAGE;
            if (j->out) {
                HIP_TRY(hipMemcpyAsync(r->hpin[b], r->snap + off, take, hipMemcpyDeviceToHost, r->xst));
            } else {
                memcpy(r->hpin[b], h + off, take);
                HIP_TRY(hipMemcpyAsync(r->snap + off, r->hpin[b], take, hipMemcpyHostToDevice, r->xst));
            }
            HIP_TRY(hipEventRecord(r->xev[b], r->xst));
            busy[b] = true;
            where[b] = h + off;
            len[b] = take;
            off += take;
        }
    }
    HIP_TRY(hipStreamSynchronize(r->xst));
    if (j->out) le64(h + payload, fnv);
    return 0;
}

void job_start(Rt * r, StateJob * j) {
    r->job = j;
    j->th = std::thread([r, j] {
        const int rc = job_run(r, j);
        std::lock_guard<std::mutex> g(j->mu);
        j->status = rc;
        if (rc == SJK_ERR_DEVICE) snprintf(j->err, sizeof(j->err), "%s", g_err);
        j->done = true;
    });
}

// wait for the job of r and take it off; its status (error text to this thread)
int job_join(Rt * r) {
    StateJob * j = r->job;
    if (!j) return 0;
    j->th.join();
    const int rc = j->status;
    if (rc == SJK_ERR_DEVICE) snprintf(g_err, sizeof(g_err), "%s", j->err);
    r->job = nullptr;
    delete j;
    return rc;
}

void rt_destroy(Rt * r) {
    if (!r) return;
    if (r->job) (void) job_join(r);
    if (r->st) (void) hipStreamSynchronize(r->st);
    if (r->xst) (void) hipStreamSynchronize(r->xst);
    for (int b = 0; b < 2; ++b) {
        if (r->dstage[b]) (void) hipFree(r->dstage[b]);
        if (r->druns[b]) (void) hipFree(r->druns[b]);
        if (r->hpin[b]) (void) hipHostFree(r->hpin[b]);
        if (r->hruns[b]) (void) hipHostFree(r->hruns[b]);
        if (r->xev[b]) (void) hipEventDestroy(r->xev[b]);
    }
    if (r->snap) (void) hipFree(r->snap);
    if (r->d_runs) (void) hipFree(r->d_runs);
    for (int i = 0; i <= RT_STORE_STREAMS; ++i) if (r->mark[i]) (void) hipEventDestroy(r->mark[i]);
    if (r->done) (void) hipEventDestroy(r->done);
    if (r->st) (void) hipStreamDestroy(r->st);
    if (r->xst) (void) hipStreamDestroy(r->xst);
    delete r;
}

}  // namespace

extern "C" {

// the checks of a state write and the header (sj_kvarn.h:1873-1929); total stream bytes in *total
static int state_header(const sj_kvarn_seq * s, void * dst, size_t dst_size, size_t * total_out) {
    const sj_kvarn_config * c = &s->cfg;
    if (!s->layers || (!dst && dst_size)) return SJKVARN_ERR_ARG;
    if (s->pol.B_pending != s->pol.B) return SJKVARN_ERR_PENDING;
    if (rt_of(s) && rt_of(s)->job) {
        sjk::set_error("an asynchronous state save or restore of this sequence is in flight");
        return SJKVARN_ERR_PENDING;
    }
    const size_t total = sj_kvarn_seq_state_size(s);
    if (dst_size < total) return SJKVARN_ERR_BUFFER;
    uint8_t * o = (uint8_t *) dst;
    memset(o, 0, SJKVARN_STATE_HEADER_BYTES);
    memcpy(o, k_state_magic, 8);
    le32(o + 8, 1); le32(o + 12, 1); le32(o + 16, SJKVARN_STATE_HEADER_BYTES);
    le32(o + 20, (uint32_t) c->head_dim); le32(o + 24, (uint32_t) c->n_head_kv); le32(o + 28, (uint32_t) c->group);
    le32(o + 32, c->sink); le32(o + 36, (uint32_t) c->sink_type); le32(o + 40, (uint32_t) c->bits_k);
    le32(o + 44, (uint32_t) c->bits_v); le32(o + 48, (uint32_t) c->body); le32(o + 52, (uint32_t) c->iters);
    le32(o + 56, (uint32_t) c->staging); le32(o + 60, c->tail); le32(o + 64, c->tail_max); le32(o + 68, c->flush_chunk);
    le32(o + 72, SJKVARN_ROTATION_HADAMARD); le32(o + 76, (uint32_t) c->head_dim);
    le64(o + 80, codebook_id(c->body, c->bits_k, c->bits_v));
    le32(o + 88, (uint32_t) s->n_layers); le32(o + 92, s->n); le32(o + 96, s->pol.B); le32(o + 100, s->pol.B_prev);
    le32(o + 104, (uint32_t) s->pol.draining);
    le64(o + 108, (uint64_t) (total - SJKVARN_STATE_HEADER_BYTES - 8));
    *total_out = total;
    return 0;
}

int sj_kvarn_seq_state_write(const sj_kvarn_seq * s, void * dst, size_t dst_size, size_t * written) {
    if (written) *written = 0;
    size_t total = 0;
    int rc = state_header(s, dst, dst_size, &total);
    if (rc) return rc;
    uint8_t * o = (uint8_t *) dst;
    Xfer x(true, o + SJKVARN_STATE_HEADER_BYTES, fnv1a(o, SJKVARN_STATE_HEADER_BYTES, FNV0));
    rc = x.open(rt_of(s));
    for (int il = 0; il < s->n_layers && !rc; ++il) rc = xfer_layer(x, &s->layers[il], s->n, s->pol.B);
    if (!rc) rc = x.finish();
    if (rc) return rc;
    le64(x.host, x.fnv);
    if (written) *written = total;
    return 0;
}

// Asynchronous save: the stream of sj_kvarn_seq_state_write. The sequence's pieces are gathered into the
// snapshot by one device launch before the call returns; a host thread then moves the snapshot to dst.
int sjk_hip_seq_state_write_begin(const sj_kvarn_seq * s, void * dst, size_t dst_size) {
    Rt * r = rt_of(s);
    if (!r) return SJKVARN_ERR_ARG;
    size_t total = 0;
    int rc = state_header(s, dst, dst_size, &total);
    if (rc) return rc;
    const size_t payload = total - SJKVARN_STATE_HEADER_BYTES - 8;
    rc = rt_xfer_buffers(r);
    if (!rc) rc = rt_snapshot(r, payload);
    if (!rc) rc = rt_after_stores(r, r->st);
    if (!rc) rc = run_copy(r, image_runs(s, s->n, s->pol.B, r->snap, true));
    if (rc) return rc;
    StateJob * j = new (std::nothrow) StateJob();
    if (!j) return SJKVARN_ERR_NOMEM;
    j->out = true;
    j->host = (uint8_t *) dst;
    j->total = total;
    j->fnv = fnv1a(dst, SJKVARN_STATE_HEADER_BYTES, FNV0);
    job_start(r, j);
    return 0;
}

static int state_peek(const void * src, size_t size, sj_kvarn_state_info * info, bool check_sum) {
    const uint8_t * p = (const uint8_t *) src;
    if (!src || !info) return SJKVARN_ERR_ARG;
    sj_kvarn_state_info t;
    memset(&t, 0, sizeof(t));
    if (size < 8) return SJKVARN_ERR_TRUNCATED;
    if (memcmp(p, k_state_magic, 8)) return SJKVARN_ERR_MAGIC;
    if (size < 16) return SJKVARN_ERR_TRUNCATED;
    t.state_version = rd32(p + 8);
    t.format_version = rd32(p + 12);
    if (t.state_version != 1) return SJKVARN_ERR_VERSION;
    if (size < SJKVARN_STATE_HEADER_BYTES + 8) return SJKVARN_ERR_TRUNCATED;
    if (rd32(p + 16) != SJKVARN_STATE_HEADER_BYTES) return SJKVARN_ERR_CORRUPT;
    const uint64_t payload = rd64(p + 108);
    if (payload > (uint64_t) (size - SJKVARN_STATE_HEADER_BYTES - 8)) return SJKVARN_ERR_TRUNCATED;
    t.total_bytes = SJKVARN_STATE_HEADER_BYTES + (size_t) payload + 8;
    if (check_sum && fnv1a(p, t.total_bytes - 8, FNV0) != rd64(p + t.total_bytes - 8)) return SJKVARN_ERR_CORRUPT;
    if (t.format_version != 1) return SJKVARN_ERR_FORMAT;
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

int sj_kvarn_state_peek(const void * src, size_t size, sj_kvarn_state_info * info) {
    return state_peek(src, size, info, true);
}

// the checks of a state read before anything is touched (sj_kvarn.h:1949-2010); the stream's checksum too
// unless check_sum is false
static int state_read_checks(sj_kvarn_seq * s, const void * src, size_t size, sj_kvarn_state_info * out, bool check_sum) {
    const sj_kvarn_config * c = &s->cfg;
    if (!s->layers) return SJKVARN_ERR_ARG;
    if (rt_of(s) && rt_of(s)->job) {
        sjk::set_error("an asynchronous state save or restore of this sequence is in flight");
        return SJKVARN_ERR_PENDING;
    }
    sj_kvarn_state_info t;
    int rc = state_peek(src, size, &t, check_sum);
    if (rc) return rc;
    if (t.cfg.head_dim != c->head_dim) return SJKVARN_ERR_HEAD_DIM;
    if (t.cfg.n_head_kv != c->n_head_kv) return SJKVARN_ERR_N_HEAD_KV;
    if (t.cfg.group != c->group) return SJKVARN_ERR_GROUP;
    if (t.cfg.sink != c->sink || t.cfg.sink_type != c->sink_type) return SJKVARN_ERR_SINK;
    if (t.cfg.bits_k != c->bits_k || t.cfg.bits_v != c->bits_v) return SJKVARN_ERR_BITS;
    if (t.cfg.body != c->body) return SJKVARN_ERR_BODY;
    if (t.cfg.iters != c->iters) return SJKVARN_ERR_ITERS;
    if (t.cfg.staging != c->staging) return SJKVARN_ERR_STAGING;
    if (t.cfg.tail != c->tail || t.cfg.tail_max != c->tail_max || t.cfg.flush_chunk != c->flush_chunk) return SJKVARN_ERR_TAIL;
    if (t.rotation != SJKVARN_ROTATION_HADAMARD || t.rotation_n != (uint32_t) c->head_dim) return SJKVARN_ERR_ROTATION;
    if (t.codebook_id != codebook_id(c->body, c->bits_k, c->bits_v)) return SJKVARN_ERR_CODEBOOK;
    if (t.n_layers != s->n_layers) return SJKVARN_ERR_N_LAYERS;
    const uint32_t S = c->sink, G = (uint32_t) c->group;
    if (t.B < S || (t.B - S) % G || t.B_prev < S || t.B_prev > t.B || (t.B_prev - S) % G || t.draining > 1 ||
        (t.B > S && t.B > t.n))
        return SJKVARN_ERR_CORRUPT;
    if (t.total_bytes != SJKVARN_STATE_HEADER_BYTES + (size_t) s->n_layers * layer_payload(c, &s->layers[0].lay, t.n, t.B) + 8)
        return SJKVARN_ERR_CORRUPT;
    const uint32_t n_rec = (t.B - S) / G;
    if (t.n > c->n_ctx || n_rec > s->layers[0].n_groups || (t.n > t.B && t.n - t.B > s->layers[0].cap))
        return SJKVARN_ERR_CAPACITY;
    if (s->pool) {
        uint32_t held = 0;
        for (uint32_t g = 0; g < s->layers[0].n_groups; ++g) held += s->blocks[g] != SJKVARN_NO_BLOCK;
        if (s->pool->n_free + held < n_rec) return SJKVARN_ERR_POOL_FULL;
    }
    *out = t;
    return 0;
}

// reset the sequence and take the blocks of the stream's records (the device table copied)
static int state_read_prepare(sj_kvarn_seq * s, const sj_kvarn_state_info & t) {
    const uint32_t n_rec = (t.B - s->cfg.sink) / (uint32_t) s->cfg.group;
    int rc = seq_reset_rc(s);
    if (!rc) rc = seq_reserve(s, 0, n_rec);
    if (!rc) rc = seq_sync_blocks(s, 0, n_rec);
    return rc;
}

static void state_read_policy(sj_kvarn_seq * s, const sj_kvarn_state_info & t) {
    s->pol.B = s->pol.B_pending = t.B;
    s->pol.B_prev = t.B_prev;
    s->pol.draining = (int) t.draining;
    s->n = t.n;
}

int sj_kvarn_seq_state_read(sj_kvarn_seq * s, const void * src, size_t size) {
    sj_kvarn_state_info t;
    int rc = state_read_checks(s, src, size, &t, true);
    if (rc) return rc;
    // everything that can fail before the sequence is touched: the transfer buffers
    Xfer x(false, (uint8_t *) src + SJKVARN_STATE_HEADER_BYTES, 0);
    rc = x.open(rt_of(s));
    if (rc) return rc;
    rc = state_read_prepare(s, t);
    for (int il = 0; il < s->n_layers && !rc; ++il) rc = xfer_layer(x, &s->layers[il], t.n, t.B);
    if (!rc) rc = x.finish();
    if (rc) return rc;        // a device failure past this point leaves the sequence reset (documented in sjk.h)
    state_read_policy(s, t);
    return 0;
}

// Asynchronous restore: the header checks now, the checksum and the upload of the payload into the snapshot on a
// host thread; sjk_hip_seq_state_finish checks the pool again, resets the sequence and scatters the snapshot.
int sjk_hip_seq_state_read_begin(sj_kvarn_seq * s, const void * src, size_t size) {
    Rt * r = rt_of(s);
    if (!r) return SJKVARN_ERR_ARG;
    sj_kvarn_state_info t;
    int rc = state_read_checks(s, src, size, &t, false);
    if (rc) return rc;
    rc = rt_xfer_buffers(r);
    if (!rc) rc = rt_snapshot(r, t.total_bytes - SJKVARN_STATE_HEADER_BYTES - 8);
    if (rc) return rc;
    StateJob * j = new (std::nothrow) StateJob();
    if (!j) return SJKVARN_ERR_NOMEM;
    j->out = false;
    j->host = (uint8_t *) src;
    j->total = t.total_bytes;
    j->n = t.n; j->B = t.B; j->B_prev = t.B_prev; j->draining = t.draining;
    job_start(r, j);
    return 0;
}

int sjk_hip_seq_state_poll(const sj_kvarn_seq * s) {
    Rt * r = rt_of(s);
    if (!r || !r->job) return 1;
    std::lock_guard<std::mutex> g(r->job->mu);
    return r->job->done ? 1 : 0;
}

static int state_job_wait(sj_kvarn_seq * s, size_t * written) {
    Rt * r = rt_of(s);
    if (written) *written = 0;
    if (!r || !r->job) return SJKVARN_ERR_ARG;
    const bool out = r->job->out;
    const size_t total = r->job->total;
    sj_kvarn_state_info t;
    memset(&t, 0, sizeof(t));
    t.n = r->job->n; t.B = r->job->B; t.B_prev = r->job->B_prev; t.draining = r->job->draining;
    int rc = job_join(r);
    if (rc) return rc;
    if (out) {
        if (written) *written = total;
        return 0;
    }
    // the restore: the pool may have changed since _begin
    const uint32_t n_rec = (t.B - s->cfg.sink) / (uint32_t) s->cfg.group;
    if (s->pool) {
        uint32_t held = 0;
        for (uint32_t g = 0; g < s->layers[0].n_groups; ++g) held += s->blocks[g] != SJKVARN_NO_BLOCK;
        if (s->pool->n_free + held < n_rec) return SJKVARN_ERR_POOL_FULL;
    }
    rc = state_read_prepare(s, t);
    if (!rc) rc = run_copy(r, image_runs(s, t.n, t.B, r->snap, false));
    if (rc) return rc;        // a device failure here leaves the sequence reset, as sj_kvarn_seq_state_read does
    state_read_policy(s, t);
    return 0;
}

int sjk_hip_seq_state_finish(sj_kvarn_seq * s, size_t * written) { return state_job_wait(s, written); }

}  // extern "C"
