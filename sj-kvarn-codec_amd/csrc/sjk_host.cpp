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
#include <cstdio>
#include <cstdlib>
#include <cstring>
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

// device buffers of one host-array call, freed when the call returns (its copies back are synchronous)
struct CallBufs {
    void * p[4] = {};
    int n = 0;
    const char * fn;
    explicit CallBufs(const char * f) : fn(f) {}
    ~CallBufs() { for (int i = 0; i < n; ++i) (void) hipFree(p[i]); }
    template <typename T> T * get(size_t bytes) {
        must_hip(hipMalloc(&p[n], bytes ? bytes : 1), fn);
        return (T *) p[n++];
    }
};

void h2d(void * d, const void * h, size_t n, const char * fn) { if (n) must_hip(hipMemcpy(d, h, n, hipMemcpyHostToDevice), fn); }
void d2h(void * h, const void * d, size_t n, const char * fn) { if (n) must_hip(hipMemcpy(h, d, n, hipMemcpyDeviceToHost), fn); }
void sync(const char * fn) { must_hip(hipDeviceSynchronize(), fn); }

uint64_t fnv1a(const void * p, size_t n, uint64_t h) {
    const uint8_t * b = (const uint8_t *) p;
    for (size_t i = 0; i < n; ++i) { h ^= b[i]; h *= 1099511628211ull; }
    return h;
}
constexpr uint64_t FNV0 = 1469598103934665603ull;

bool frag_side(const sj_kvarn_layout * l, int bits) {
    return l->body == SJKVARN_BODY_SCALAR && bits == 4 && l->D % 16 == 0 && l->G % 16 == 0;
}

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

// A layout the device seal is not built for (sjk_hip_supported) leaves rec as it is, with a message: there is
// no status to return and no CPU path.
void sj_kvarn_seal_group(const sj_kvarn_layout * l, const uint16_t * K, const uint16_t * V, size_t row_stride, int iters,
                         uint8_t * rec, void * work) {
    (void) work;
    if (!sjk_hip_supported(l)) {
        fprintf(stderr, "libsjk: sj_kvarn_seal_group: layout D=%d G=%d not supported by the HIP seal (D 128/256, "
                        "G 128); record left unwritten\n", l->D, l->G);
        return;
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

// fp16 staging of any D: the row kernel's widths for D in {128, 256, 512}, else rows of 128 (or fewer) values
void sj_kvarn_stage_row(int staging, const float * x_rot, void * dst, int D) {
    if (staging == SJKVARN_STAGING_TQ6_0) { sj_kvarn_tq6_quantize_row(x_rot, (sj_kvarn_tq6_block *) dst, D); return; }
    if (D <= 0) return;
    CallBufs b("sj_kvarn_stage_row");
    const size_t ob = sj_kvarn_stage_row_bytes(staging, D);
    float * dx = b.get<float>((size_t) D * 4);
    uint8_t * dy = b.get<uint8_t>(ob);
    h2d(dx, x_rot, (size_t) D * 4, b.fn);
    if (D == 128 || D == 256 || D == 512) {
        must(sjk_hip_stage(staging, dx, dy, D, ob, 1, nullptr), b.fn);
    } else {
        // fp16 staging converts each value on its own: the row is cut into pieces the kernel takes
        for (int o = 0; o < D; o += 128) {
            const int w = D - o < 128 ? D - o : 128;
            must(sjk_hip_stage(staging, dx + o, dy + 2 * o, w, 2 * (size_t) w, 1, nullptr), b.fn);
        }
    }
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

int sj_kvarn_layer_init(sj_kvarn_layer * L, const sj_kvarn_config * cfg) { return layer_setup(L, cfg, 1, nullptr); }

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
    sync("sj_kvarn_layer_store");
}

void sj_kvarn_layer_seal(sj_kvarn_layer * L, uint32_t B_from, uint32_t B_to) {
    const sjk_hip_view v = sjk_layer_view(L);
    must(sjk_hip_commit(&v, 1, B_from, B_to, L->cfg.iters, nullptr), "sj_kvarn_layer_seal");
    sync("sj_kvarn_layer_seal");
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

// zero every run in one launch (synchronous, as the reference's memsets)
static int zero_runs(const std::vector<sjk::CopyRun> & runs) {
    if (runs.empty()) return 0;
    sjk::CopyRun * d = nullptr;
    HIP_TRY(hipMalloc((void **) &d, runs.size() * sizeof(sjk::CopyRun)));
    int rc = 0;
    if (hipMemcpy(d, runs.data(), runs.size() * sizeof(sjk::CopyRun), hipMemcpyHostToDevice) != hipSuccess ||
        sjk::sjk_zero_runs(d, (int) runs.size(), nullptr) || hipStreamSynchronize(nullptr) != hipSuccess)
        rc = hip_fail(hipGetLastError(), "truncate scrub");
    (void) hipFree(d);
    return rc;
}

void sj_kvarn_layer_truncate(sj_kvarn_layer * L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume) {
    std::vector<sjk::CopyRun> runs;
    truncate_runs(L, B_old, B_new, n_old, resume, runs);
    must(zero_runs(runs), "sj_kvarn_layer_truncate");
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

// the device copy of a sequence's block table lives in layers[0].work (shared by every layer)
static int seq_sync_blocks(sj_kvarn_seq * s) {
    if (!s->pool) return 0;
    HIP_TRY(hipMemcpy(s->layers[0].work, s->blocks, (size_t) s->layers[0].n_groups * 4, hipMemcpyHostToDevice));
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
    sj_kvarn_policy_init(&s->pol, cfg->sink, cfg->tail, cfg->tail_max, (uint32_t) cfg->group, cfg->flush_chunk);
    s->n = 0;
    return 0;
}

static void seq_release(sj_kvarn_seq * s, uint32_t g0, uint32_t g1) {
    if (!s->pool || !s->blocks) return;
    for (uint32_t g = g0; g < g1 && g < s->layers[0].n_groups; ++g) {
        sj_kvarn_pool_release(s->pool, s->blocks[g]);
        s->blocks[g] = SJKVARN_NO_BLOCK;
    }
    must(seq_sync_blocks(s), "sj_kvarn_seq (block table)");
}

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
    return seq_sync_blocks(s);
}

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
static void seq_scrub(sj_kvarn_seq * s, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume, const char * fn) {
    std::vector<sjk::CopyRun> runs;
    for (int il = 0; il < s->n_layers; ++il) truncate_runs(&s->layers[il], B_old, B_new, n_old, resume, runs);
    must(zero_runs(runs), fn);
}

void sj_kvarn_seq_reset(sj_kvarn_seq * s) {
    seq_scrub(s, s->pol.B, s->cfg.sink, s->n, 0, "sj_kvarn_seq_reset");
    seq_release(s, 0, s->layers[0].n_groups);
    sj_kvarn_policy_reset(&s->pol);
    s->n = 0;
}

// seal [B, B_pending) in every layer with one launch, then commit; a failure leaves the sequence unchanged
static int seq_seal_commit(sj_kvarn_seq * s, const sj_kvarn_policy * before) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group;
    if (s->pol.B_pending > s->pol.B) {
        int rc = seq_reserve(s, (s->pol.B - S) / G, (s->pol.B_pending - S) / G);
        if (rc) { s->pol = *before; return rc; }
        sjk_hip_view views[64];
        for (int il = 0; il < s->n_layers; il += 64) {
            const int nl = s->n_layers - il < 64 ? s->n_layers - il : 64;
            for (int k = 0; k < nl; ++k) views[k] = sjk_layer_view(&s->layers[il + k]);
            rc = sjk_hip_commit(views, nl, s->pol.B, s->pol.B_pending, s->cfg.iters, nullptr);
            if (rc) { s->pol = *before; return rc; }
        }
        if (hipDeviceSynchronize() != hipSuccess) { s->pol = *before; return SJK_ERR_DEVICE; }
    }
    sj_kvarn_policy_commit(&s->pol);
    return 0;
}

int sj_kvarn_seq_begin_ubatch(sj_kvarn_seq * s, uint32_t pos0, uint32_t n_tokens) {
    const sj_kvarn_policy before = s->pol;
    if (pos0 > s->n) return SJKVARN_ERR_ARG;
    sj_kvarn_policy_begin_ubatch(&s->pol, pos0, n_tokens);
    return seq_seal_commit(s, &before);
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
    return seq_seal_commit(s, &before);
}

uint32_t sj_kvarn_seq_truncate(sj_kvarn_seq * s, uint32_t pos) {
    const uint32_t S = s->cfg.sink, G = (uint32_t) s->cfg.group, B_old = s->pol.B, n_old = s->n;
    const uint32_t r = sj_kvarn_policy_truncate(&s->pol, pos, nullptr);
    if (r == SJKVARN_NO_POS) return r;
    seq_scrub(s, B_old, s->pol.B, n_old, r, "sj_kvarn_seq_truncate");
    if (s->pol.B < B_old) seq_release(s, (s->pol.B - S) / G, (B_old - S) / G);
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

// The device pieces of a state stream (sink, records, ring rows of every layer, in stream order) move in
// chunks through two device staging buffers and two pinned host buffers, on a stream of the call's own:
// writing, chunk k is gathered on the device (one sjk_copy_runs launch) and copied to pinned memory while the
// host copies chunk k - 1 into the caller's buffer and extends the stream's FNV-1a checksum over it; reading,
// the host fills the pinned buffer of chunk k while the device copies in and scatters chunk k - 1.
// Contiguous pieces merge into one run. Every buffer is allocated by open(), before the sequence is touched.
constexpr size_t XFER_STAGE = (size_t) 32 << 20;   // stream bytes per chunk
constexpr size_t XFER_RUNS = 1 << 15;              // runs per chunk

struct Xfer {
    bool out;                            // device -> host stream (state write)
    uint8_t * host;                      // stream byte of the next chunk's first byte
    uint64_t fnv = 0;                    // write: checksum of the stream bytes handed to the host so far
    uint8_t * dstage[2] = {};
    sjk::CopyRun * druns[2] = {};
    uint8_t * hpin[2] = {};
    sjk::CopyRun * hruns[2] = {};
    hipStream_t st = nullptr;
    hipEvent_t ev[2] = {};
    bool busy[2] = {};                   // chunk in flight in buffer b
    uint8_t * dest[2] = {};              // write: where chunk b goes in the caller's buffer
    size_t len[2] = {};
    int cur = 0;                         // buffer of the chunk being assembled
    size_t fill = 0, n_runs = 0;

    Xfer(bool o, uint8_t * h, uint64_t f) : out(o), host(h), fnv(f) {}
    Xfer(const Xfer &) = delete;
    Xfer & operator=(const Xfer &) = delete;

    int open() {
        HIP_TRY(hipStreamCreate(&st));
        for (int b = 0; b < 2; ++b) {
            HIP_TRY(hipMalloc((void **) &dstage[b], XFER_STAGE));
            HIP_TRY(hipMalloc((void **) &druns[b], XFER_RUNS * sizeof(sjk::CopyRun)));
            HIP_TRY(hipHostMalloc((void **) &hpin[b], XFER_STAGE, hipHostMallocDefault));
            HIP_TRY(hipHostMalloc((void **) &hruns[b], XFER_RUNS * sizeof(sjk::CopyRun), hipHostMallocDefault));
            HIP_TRY(hipEventCreateWithFlags(&ev[b], hipEventDisableTiming));
        }
        return 0;
    }

    ~Xfer() {
        if (st) (void) hipStreamSynchronize(st);
        for (int b = 0; b < 2; ++b) {
            if (dstage[b]) (void) hipFree(dstage[b]);
            if (druns[b]) (void) hipFree(druns[b]);
            if (hpin[b]) (void) hipHostFree(hpin[b]);
            if (hruns[b]) (void) hipHostFree(hruns[b]);
            if (ev[b]) (void) hipEventDestroy(ev[b]);
        }
        if (st) (void) hipStreamDestroy(st);
    }

    // wait for the chunk in buffer b; writing, hand its bytes to the caller and the checksum
    int retire(int b) {
        if (!busy[b]) return 0;
        HIP_TRY(hipEventSynchronize(ev[b]));
        if (out) {
            memcpy(dest[b], hpin[b], len[b]);
            fnv = fnv1a(dest[b], len[b], fnv);
        }
        busy[b] = false;
        return 0;
    }

    int region(const uint8_t * dev, size_t bytes) {
        while (bytes) {
            const size_t take = bytes < XFER_STAGE - fill ? bytes : XFER_STAGE - fill;
            const uint64_t d = (uint64_t) (uintptr_t) dev, sg = (uint64_t) (uintptr_t) (dstage[cur] + fill);
            const sjk::CopyRun r = out ? sjk::CopyRun{d, sg, take} : sjk::CopyRun{sg, d, take};
            sjk::CopyRun * rs = hruns[cur];
            if (n_runs && rs[n_runs - 1].src + rs[n_runs - 1].bytes == r.src && rs[n_runs - 1].dst + rs[n_runs - 1].bytes == r.dst)
                rs[n_runs - 1].bytes += take;
            else
                rs[n_runs++] = r;
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
            memcpy(hpin[b], host, fill);
            HIP_TRY(hipMemcpyAsync(dstage[b], hpin[b], fill, hipMemcpyHostToDevice, st));
        }
        HIP_TRY(hipMemcpyAsync(druns[b], hruns[b], n_runs * sizeof(sjk::CopyRun), hipMemcpyHostToDevice, st));
        if (sjk::sjk_copy_runs(druns[b], (int) n_runs, st)) return hip_fail(hipGetLastError(), "sjk_copy_runs");
        if (out) HIP_TRY(hipMemcpyAsync(hpin[b], dstage[b], fill, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipEventRecord(ev[b], st));
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

// the pieces of one layer in stream order: sink rows [0, min(n, S)), records of [S, B), ring rows [B, n)
static int xfer_layer(Xfer & x, const sj_kvarn_layer * L, uint32_t n, uint32_t B) {
    const uint32_t S = L->cfg.sink, G = (uint32_t) L->cfg.group;
    const int H = L->cfg.n_head_kv;
    const uint32_t ns = n < S ? n : S;
    int rc = x.region(L->sink, (size_t) ns * H * sink_entry_bytes(L));
    const uint32_t n_rec = (B - S) / G;
    const size_t gb = (size_t) H * L->lay.bytes;
    for (uint32_t g = 0; g < n_rec && !rc; ++g) rc = x.region(sj_kvarn_layer_record(L, g, 0), gb);
    const size_t re = (size_t) H * 2 * L->stage_bytes;
    for (uint32_t pos = B; pos < n && !rc; ++pos) rc = x.region(ring_entry(L, pos, 0), re);
    return rc;
}

int sj_kvarn_seq_state_write(const sj_kvarn_seq * s, void * dst, size_t dst_size, size_t * written) {
    const sj_kvarn_config * c = &s->cfg;
    if (written) *written = 0;
    if (!s->layers || (!dst && dst_size)) return SJKVARN_ERR_ARG;
    if (s->pol.B_pending != s->pol.B) return SJKVARN_ERR_PENDING;
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
    Xfer x(true, o + SJKVARN_STATE_HEADER_BYTES, fnv1a(o, SJKVARN_STATE_HEADER_BYTES, FNV0));
    int rc = x.open();
    for (int il = 0; il < s->n_layers && !rc; ++il) rc = xfer_layer(x, &s->layers[il], s->n, s->pol.B);
    if (!rc) rc = x.finish();
    if (rc) return rc;
    le64(x.host, x.fnv);
    if (written) *written = total;
    return 0;
}

int sj_kvarn_state_peek(const void * src, size_t size, sj_kvarn_state_info * info) {
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
    if (fnv1a(p, t.total_bytes - 8, FNV0) != rd64(p + t.total_bytes - 8)) return SJKVARN_ERR_CORRUPT;
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

int sj_kvarn_seq_state_read(sj_kvarn_seq * s, const void * src, size_t size) {
    const sj_kvarn_config * c = &s->cfg;
    if (!s->layers) return SJKVARN_ERR_ARG;
    sj_kvarn_state_info t;
    int rc = sj_kvarn_state_peek(src, size, &t);
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
    // everything that can fail before the sequence is touched: the transfer buffers
    Xfer x(false, (uint8_t *) src + SJKVARN_STATE_HEADER_BYTES, 0);
    rc = x.open();
    if (rc) return rc;
    sj_kvarn_seq_reset(s);
    rc = seq_reserve(s, 0, n_rec);
    if (rc) return rc;
    for (int il = 0; il < s->n_layers && !rc; ++il) rc = xfer_layer(x, &s->layers[il], t.n, t.B);
    if (!rc) rc = x.finish();
    if (rc) return rc;        // a device failure past this point leaves the sequence reset (documented in sjk.h)
    s->pol.B = s->pol.B_pending = t.B;
    s->pol.B_prev = t.B_prev;
    s->pol.draining = (int) t.draining;
    s->n = t.n;
    return 0;
}

}  // extern "C"
