/* sjk.h - C ABI of the MI355X (gfx950) SJ-KVaRN codec library, libsjk.so.
 *
 * Two layers, both plain C (no torch or HIP C++ types; hipStream_t is passed as void *):
 *
 * 1. The sj_kvarn.h API, same names, types and argument meaning (reference sj_kvarn.h:177-453), so
 *    an engine written against the reference header links against this library unchanged. The codec
 *    routines run as HIP kernels on the current device; the cache objects (layer, pool, sequence)
 *    keep their sink, staging ring and sealed body in device memory (HBM) with the reference's byte
 *    layout, while the rows, queries and outputs handed across the API stay host arrays as in the
 *    reference. One documented difference: sj_kvarn_layer_record() and the ring/sink/body members
 *    of sj_kvarn_layer / sj_kvarn_pool are DEVICE addresses.
 *
 * 2. sjk_hip_*: the device entry points the engine's hot path calls (device pointers, explicit
 *    stream, batched over records, rows, positions and layers). They replace the reference's CUDA
 *    kernels and launcher in sj_kvarn_cuda.cuh:27-151 and the per-layer loops of sj_kvarn.h.
 *
 * Status codes: the SJKVARN_* space of the reference (sj_kvarn.h:332-361) plus SJK_ERR_DEVICE
 * (a HIP call failed) and SJK_ERR_UNSUPPORTED (a shape the kernels are not built for).
 * Every function that returns a status leaves its outputs untouched when it fails before launching.
 */
#ifndef SJK_H
#define SJK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- format constants (sj_kvarn.h:114-131) ---- */
#define SJKVARN_GROUP_DEFAULT     128
#define SJKVARN_SINK_DEFAULT      128
#define SJKVARN_TAIL_DEFAULT      4096
#define SJKVARN_TAIL_MAX_DEFAULT  8192
#define SJKVARN_ITERS_DEFAULT     16
#define SJKVARN_RED_LANES         8
#define SJKVARN_TQ6_QK            128
#define SJKVARN_TQ6_BLOCK_BYTES   98
#define SJKVARN_TRELLIS_SEQ       128
#define SJKVARN_TRELLIS_HIST_BITS 6
#define SJKVARN_TRELLIS_NSTATE    64
#define SJKVARN_NO_POS            UINT32_MAX
#define SJKVARN_NO_BLOCK          UINT32_MAX
#define SJKVARN_STATE_HEADER_BYTES 128
#define SJKVARN_ROTATION_HADAMARD 1

typedef enum sj_kvarn_body { SJKVARN_BODY_SCALAR = 0, SJKVARN_BODY_TRELLIS = 1, SJKVARN_BODY_AUTO = 2 } sj_kvarn_body;
typedef enum sj_kvarn_staging { SJKVARN_STAGING_TQ6_0 = 0, SJKVARN_STAGING_F16 = 1 } sj_kvarn_staging;
typedef enum sj_kvarn_sink_type { SJKVARN_SINK_F16 = 0, SJKVARN_SINK_INHERIT = 1 } sj_kvarn_sink_type;

/* 98-byte staging block (sj_kvarn.h:146-154) */
typedef struct sj_kvarn_tq6_block {
    uint16_t norm;
    uint8_t  qs[64];
    uint8_t  qh[32];
} sj_kvarn_tq6_block;

/* record layout (sj_kvarn.h:170-175) */
typedef struct sj_kvarn_layout {
    int D, G, bits_k, bits_v, body;
    uint32_t k_payload, v_payload;
    uint32_t k_scale, k_zero, k_tok, v_ch, v_scale, v_zero;
    uint32_t bytes;
} sj_kvarn_layout;

/* journal policy (sj_kvarn.h:228-234) */
typedef struct sj_kvarn_policy {
    uint32_t sink, tail, tail_max, group, flush_chunk;
    uint32_t B, B_prev, B_pending;
    int      draining;
} sj_kvarn_policy;

/* cache configuration (sj_kvarn.h:279-291) */
typedef struct sj_kvarn_config {
    int      head_dim, n_head_kv, group, bits_k, bits_v, body, iters, staging, sink_type;
    uint32_t sink, tail, tail_max, flush_chunk, n_ubatch, n_ctx;
} sj_kvarn_config;

/* per-layer cache (sj_kvarn.h:293-309); ring, sink and body are device memory here */
typedef struct sj_kvarn_layer {
    sj_kvarn_config cfg;
    sj_kvarn_layout lay;
    uint32_t cap, n_groups;
    size_t   stage_bytes;
    uint8_t * ring;            /* device: [cap][n_head_kv][K row | V row] */
    uint8_t * sink;            /* device: f16 [sink][n_head_kv][K D | V D] fp16, inherit: staging rows */
    uint8_t * body;            /* device: [n_groups][n_head_kv][lay.bytes] (or a pool slab) */
    void    * work;            /* the HIP seal needs no workspace: pool mode keeps the device copy of the
                                  sequence's block table here, NULL otherwise */
    uint16_t * kstage;         /* DEVICE workspace of the layer's attention calls (sjk_hip_workspace_bytes;
                                  the layers of a sequence share their first layer's), not host staging */
    uint16_t * vstage;         /* the library's private runtime of the cache object (a layer of layer_init, or a
                                  sequence, kept with its first layer): its stream, truncation run table and state
                                  transfer buffers; opaque, set by init, freed by free (the device seal reads the
                                  ring directly and needs no host staging) */
    const uint32_t * blocks;   /* host block table (pool mode), NULL = contiguous body */
    int       owns_body;
} sj_kvarn_layer;

/* status codes (sj_kvarn.h:333-359) */
enum {
    SJKVARN_OK = 0,
    SJKVARN_ERR_ARG = -100, SJKVARN_ERR_NOMEM = -101, SJKVARN_ERR_BUFFER = -102, SJKVARN_ERR_TRUNCATED = -103,
    SJKVARN_ERR_MAGIC = -104, SJKVARN_ERR_VERSION = -105, SJKVARN_ERR_FORMAT = -106, SJKVARN_ERR_CORRUPT = -107,
    SJKVARN_ERR_PENDING = -108, SJKVARN_ERR_CAPACITY = -109, SJKVARN_ERR_POOL_FULL = -110,
    SJKVARN_ERR_HEAD_DIM = -120, SJKVARN_ERR_N_HEAD_KV = -121, SJKVARN_ERR_GROUP = -122, SJKVARN_ERR_SINK = -123,
    SJKVARN_ERR_BITS = -124, SJKVARN_ERR_BODY = -125, SJKVARN_ERR_ITERS = -126, SJKVARN_ERR_STAGING = -127,
    SJKVARN_ERR_TAIL = -128, SJKVARN_ERR_ROTATION = -129, SJKVARN_ERR_CODEBOOK = -130, SJKVARN_ERR_N_LAYERS = -131,
    /* this library only: */
    SJK_ERR_DEVICE = -140,      /* a HIP runtime call or kernel launch failed */
    SJK_ERR_UNSUPPORTED = -141  /* shape outside what the kernels are built for (see sjk_hip_supported) */
};

/* ---- pool / sequence / state (sj_kvarn.h:366-442) ---- */
typedef struct sj_kvarn_pool {
    sj_kvarn_config cfg;
    sj_kvarn_layout lay;
    int       n_layers;
    uint32_t  n_blocks;
    uint8_t * body;            /* device: [n_layers][n_blocks][n_head_kv][lay.bytes] */
    uint32_t * free_ids;       /* host */
    uint32_t  n_free;
} sj_kvarn_pool;

typedef struct sj_kvarn_seq {
    sj_kvarn_config  cfg;
    int              n_layers;
    sj_kvarn_layer * layers;
    sj_kvarn_policy  pol;
    uint32_t         n;
    sj_kvarn_pool  * pool;
    uint32_t       * blocks;   /* host block table */
} sj_kvarn_seq;

typedef struct sj_kvarn_state_info {
    uint32_t state_version, format_version;
    sj_kvarn_config cfg;
    uint32_t rotation, rotation_n;
    uint64_t codebook_id;
    int      n_layers;
    uint32_t n, B, B_prev, draining;
    size_t   total_bytes;
} sj_kvarn_state_info;

/* ================================================================================================ */
/* 1. sj_kvarn.h API                                                                                */
/* ================================================================================================ */

/* fp16 conversion, host scalar helpers (sj_kvarn.h:181-182) */
uint16_t sj_kvarn_f32_to_f16(float f);
float    sj_kvarn_f16_to_f32(uint16_t h);

/* rotation (sj_kvarn.h:184-185): runs on the device, for any power-of-two n (the reference's stages read past
 * the end of x for other n; here such a call leaves x as it is) */
void sj_kvarn_hadamard(float * x, int n);
void sj_kvarn_rotate_heads(float * x, int n_heads, int head_dim);

/* record layout (sj_kvarn.h:188-195): host integer logic */
int      sj_kvarn_body_resolve(int body, int bits_k, int bits_v);
int      sj_kvarn_layout_init(sj_kvarn_layout * l, int D, int G, int bits_k, int bits_v, int body);
size_t   sj_kvarn_record_bytes(int D, int G, int bits_k, int bits_v);
double   sj_kvarn_body_bits_per_element(const sj_kvarn_layout * l);
uint32_t sj_kvarn_code_bit(const sj_kvarn_layout * l, int t, int d, int is_v);
int      sj_kvarn_k_ch_idx(const sj_kvarn_layout * l, int d);
int      sj_kvarn_v_ch_idx(const sj_kvarn_layout * l, int d);

/* seal / decode (sj_kvarn.h:199-208): run on the device; rows, rec and out are host arrays.
 * The HIP seal needs no workspace: sj_kvarn_seal_workspace_bytes() returns the reference's figure
 * for ABI compatibility and `work` is ignored. */
size_t sj_kvarn_seal_workspace_bytes(const sj_kvarn_layout * l);
void   sj_kvarn_seal_group(const sj_kvarn_layout * l, const uint16_t * K, const uint16_t * V, size_t row_stride,
                           int iters, uint8_t * rec, void * work);
void   sj_kvarn_decode_k_row(const sj_kvarn_layout * l, const uint8_t * rec, int t, float * out);
void   sj_kvarn_decode_v_row(const sj_kvarn_layout * l, const uint8_t * rec, int t, float * out);

/* staging (sj_kvarn.h:212-216): run on the device */
void   sj_kvarn_tq6_quantize_row(const float * x, sj_kvarn_tq6_block * y, int n);
void   sj_kvarn_tq6_dequantize_row(const sj_kvarn_tq6_block * y, float * x, int n);
size_t sj_kvarn_stage_row_bytes(int staging, int D);
void   sj_kvarn_stage_row(int staging, const float * x_rot, void * dst, int D);
void   sj_kvarn_unstage_row(int staging, const void * src, float * x_rot, int D);

/* attention helpers (sj_kvarn.h:220-222): run on the device */
void sj_kvarn_record_scores(const sj_kvarn_layout * l, const uint8_t * rec, const float * q, int n, float * scores);
void sj_kvarn_record_accum_v(const sj_kvarn_layout * l, const uint8_t * rec, const float * w, int n, float * acc);

/* journal policy, truncation, ring (sj_kvarn.h:236-274): host integer logic */
void     sj_kvarn_policy_init(sj_kvarn_policy * p, uint32_t sink, uint32_t tail, uint32_t tail_max, uint32_t group,
                              uint32_t flush_chunk);
void     sj_kvarn_policy_reset(sj_kvarn_policy * p);
uint32_t sj_kvarn_policy_begin_ubatch(sj_kvarn_policy * p, uint32_t pos0, uint32_t n_tokens);
void     sj_kvarn_policy_commit(sj_kvarn_policy * p);
uint32_t sj_kvarn_policy_idle(sj_kvarn_policy * p, uint32_t end, uint32_t keep_recent);
uint32_t sj_kvarn_group_floor(uint32_t sink, uint32_t group, uint32_t pos);
uint32_t sj_kvarn_policy_trunc_floor(const sj_kvarn_policy * p, uint32_t pos);
uint32_t sj_kvarn_policy_truncate(sj_kvarn_policy * p, uint32_t pos, uint32_t * n_dropped);
uint32_t sj_kvarn_ring_capacity(uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t n_ubatch);
uint32_t sj_kvarn_ring_slot(uint32_t sink, uint32_t cap, uint32_t pos);

/* per-layer cache (sj_kvarn.h:311-330): device-resident buffers, host rows at the API */
sj_kvarn_config sj_kvarn_config_default(int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch);
int       sj_kvarn_layer_init(sj_kvarn_layer * L, const sj_kvarn_config * cfg);
void      sj_kvarn_layer_free(sj_kvarn_layer * L);
void      sj_kvarn_layer_store(sj_kvarn_layer * L, uint32_t pos, const float * k_rot, const float * v_rot);
void      sj_kvarn_layer_seal(sj_kvarn_layer * L, uint32_t B_from, uint32_t B_to);
void      sj_kvarn_layer_kv_row(const sj_kvarn_layer * L, uint32_t B, uint32_t pos, int h, float * k, float * v);
void      sj_kvarn_layer_attend_row(const sj_kvarn_layer * L, uint32_t B, uint32_t N, const float * q_rot, int h,
                                    uint32_t qpos, float scale, float * out_rot);
uint8_t * sj_kvarn_layer_record(const sj_kvarn_layer * L, uint32_t g, int h);   /* DEVICE address */
void      sj_kvarn_layer_truncate(sj_kvarn_layer * L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume);
const char * sj_kvarn_strerror(int code);

/* pool / sequence / state (sj_kvarn.h:378-442) */
int      sj_kvarn_pool_init(sj_kvarn_pool * pool, const sj_kvarn_config * cfg, int n_layers, uint32_t n_blocks);
void     sj_kvarn_pool_free(sj_kvarn_pool * pool);
uint32_t sj_kvarn_pool_alloc(sj_kvarn_pool * pool);
void     sj_kvarn_pool_release(sj_kvarn_pool * pool, uint32_t id);
int      sj_kvarn_seq_init(sj_kvarn_seq * s, const sj_kvarn_config * cfg, int n_layers, sj_kvarn_pool * pool);
void     sj_kvarn_seq_free(sj_kvarn_seq * s);
void     sj_kvarn_seq_reset(sj_kvarn_seq * s);
/* seq_begin_ubatch / seq_idle: a due commit seals [B, B_pending) of every layer in one launch on the sequence's own
 * stream, after the work enqueued on the null stream and on the streams its device stores used
 * (sjk_hip_seq_store, _batch), and waits for that seal only, not for the rest of the device. */
int      sj_kvarn_seq_begin_ubatch(sj_kvarn_seq * s, uint32_t pos0, uint32_t n_tokens);
void     sj_kvarn_seq_store(sj_kvarn_seq * s, uint32_t pos, const float * k_rot, const float * v_rot);
int      sj_kvarn_seq_idle(sj_kvarn_seq * s, uint32_t keep_recent);
uint32_t sj_kvarn_seq_truncate(sj_kvarn_seq * s, uint32_t pos);
void     sj_kvarn_seq_attend_row(const sj_kvarn_seq * s, int il, const float * q_rot, int h, uint32_t qpos, float scale,
                                 float * out_rot);
size_t   sj_kvarn_seq_state_size(const sj_kvarn_seq * s);
size_t   sj_kvarn_state_size_max(const sj_kvarn_config * cfg, int n_layers);
int      sj_kvarn_seq_state_write(const sj_kvarn_seq * s, void * dst, size_t dst_size, size_t * written);
int      sj_kvarn_state_peek(const void * src, size_t size, sj_kvarn_state_info * info);
/* seq_state_read: every check of the reference (sj_kvarn.h:1949-2034) runs, and the transfer buffers are
 * allocated, before the sequence is touched; a rejected stream leaves it unchanged. A device failure during
 * the copy itself returns SJK_ERR_DEVICE with the sequence reset (empty). */
int      sj_kvarn_seq_state_read(sj_kvarn_seq * s, const void * src, size_t size);

/* ================================================================================================ */
/* 2. device entry points (device pointers, stream = hipStream_t or NULL for the null stream)       */
/* ================================================================================================ */

/* Device view of one layer's cache, byte layout of sj_kvarn_layer (sj_kvarn_cuda.cuh:27-42), plus
 * an optional device block table: record (g, h) at body + ((blocks ? blocks[g] : g)*n_head_kv + h)*lay.bytes. */
typedef struct sjk_hip_view {
    sj_kvarn_layout lay;
    int       n_head_kv;
    int       staging;
    int       sink_type;
    uint32_t  S, cap;
    size_t    stage_bytes;
    uint8_t * sink;
    uint8_t * ring;
    uint8_t * body;
    const uint32_t * blocks;
    void    * work;            /* device workspace of the attention calls on this view (their partial results, the plan
                                  of a 4/4 sjk_hip_attend_dyn call, the staging of the host-array layer calls):
                                  sjk_hip_workspace_bytes() bytes. sjk_layer_view
                                  fills it with the layer's own; a hand-built view brings one. Calls that
                                  share a workspace must be ordered (one stream, or the caller's
                                  synchronisation), as for the cache itself. */
    size_t    work_bytes;
} sjk_hip_view;

/* 1 when the kernels are built for this layout (D in {128, 256}, G = 128), else 0 */
int sjk_hip_supported(const sj_kvarn_layout * l);

/* Bytes of device workspace that attention calls on a view with this layout and KV head count need
 * (sjk_hip_view.work); sized on the current device. No counterpart in the reference (whose attention keeps its
 * state in registers of one thread per row and head, sj_kvarn_cuda.cuh:102-135). */
size_t sjk_hip_workspace_bytes(const sj_kvarn_layout * l, int n_head_kv);

/* Seal n_groups*n_head_kv records from fp16 rows: record r = g*n_head_kv + h reads the G rows
 * k + g*G*row_stride + h*D (+ t*row_stride) and writes body + r*l->bytes.
 * Replaces sj_kvarn_cuda_seal (sj_kvarn_cuda.cuh:142-151); needs no workspace. */
int sjk_hip_seal(const sj_kvarn_layout * l, const uint16_t * d_k, const uint16_t * d_v, size_t row_stride,
                 int n_head_kv, int n_groups, int iters, uint8_t * d_body, void * stream);

/* Decode n_rec records to fp32 rows out_k/out_v [n_rec][G][D] (sj_kvarn_cuda.cuh:57-66). */
int sjk_hip_decode(const sj_kvarn_layout * l, const uint8_t * d_body, int n_rec, float * d_out_k, float * d_out_v,
                   void * stream);

/* Stage / unstage n_rows rows of D values (sj_kvarn_cuda.cuh:68-80). */
int sjk_hip_stage(int staging, const float * d_x, uint8_t * d_dst, int D, size_t dst_row_bytes, int n_rows, void * stream);
int sjk_hip_unstage(int staging, const uint8_t * d_src, size_t src_row_bytes, float * d_x, int D, int n_rows,
                    void * stream);

/* In-place orthonormal Hadamard of n_rows rows of D floats, D any power of two (sj_kvarn_rotate_heads,
 * sj_kvarn.h:754-759); SJKVARN_ERR_ARG for other D. */
int sjk_hip_rotate(float * d_x, int n_rows, int D, void * stream);

/* The rotation folded into the projection weights at load time (the reference's INTEGRATION_LLAMACPP.md:46: "the
 * rotation can also be folded into the Q/K/V/O weights at load time"; the fork's fused Q / output rotation,
 * README.md:45-54), so that a decode step needs no sj_kvarn_rotate_heads on q, k, v and none on the attention
 * output. R = the Hadamard of sj_kvarn_hadamard (H / sqrt(D), symmetric, its own inverse); device memory, fp32,
 * row-major, in place, any power-of-two D.
 * sjk_hip_fold_rotation_out: W is [n_heads * head_dim][cols] (W_q, W_k or W_v; a bias with cols = 1): every column's
 *   head_dim-blocks become R times them, W' = blockdiag(R) W, so W' x is the rotated projection, value for value the
 *   reference's sj_kvarn_rotate_heads(W x) up to the rounding of the product (then store with rotate = 0).
 * sjk_hip_fold_rotation_in: W is [rows][n_heads * head_dim] (W_o): every row's head segments become R times them,
 *   W' = W blockdiag(R), so W' takes the attention's rotated output directly.
 * Each folded vector is bit for bit sj_kvarn_hadamard of the original. No counterpart function in the reference,
 * which describes the folding without shipping it. */
int sjk_hip_fold_rotation_out(float * d_w, int n_heads, int head_dim, int cols, void * stream);
int sjk_hip_fold_rotation_in(float * d_w, int rows, int n_heads, int head_dim, void * stream);

/* Append n_pos positions pos0.. to a layer (sj_kvarn_layer_store, sj_kvarn.h:1475-1492, batched):
 * d_k, d_v are [n_pos][n_head_kv][D] floats. rotate != 0 applies the Hadamard first (the engine's
 * sj_kvarn_rotate_heads fused into the append); rotate == 0 expects rotated rows. */
int sjk_hip_layer_store(const sjk_hip_view * v, uint32_t pos0, uint32_t n_pos, const float * d_k, const float * d_v,
                        int rotate, void * stream);

/* sjk_hip_layer_store with pos0 = d_desc[SJK_DESC_QPOS0] read on the device when the kernel runs, so a captured
 * HIP graph stores every decode step's rows (the reference's staged write ggml_set_rows_stage,
 * INTEGRATION_LLAMACPP.md:47, whose row indices are a graph input). A negative entry stores nothing. */
int sjk_hip_layer_store_dyn(const sjk_hip_view * v, const int32_t * d_desc, uint32_t n_pos, const float * d_k,
                            const float * d_v, int rotate, void * stream);

/* Commit: seal groups [B_from, B_to) of every KV head of n_layers layers straight out of their
 * staging rings in one launch (sj_kvarn_layer_seal, sj_kvarn.h:1494-1514, for each layer). */
int sjk_hip_commit(const sjk_hip_view * views, int n_layers, uint32_t B_from, uint32_t B_to, int iters, void * stream);

/* Run-time descriptor of a commit: 16 int32 in device memory, at the indices of the reference's seal_dyn
 * descriptor (INTEGRATION_LLAMACPP.md:51-71). sjk_hip_commit_dyn reads SJK_DESC_B_OLD and SJK_DESC_B. */
enum {
    SJK_DESC_S = 0, SJK_DESC_CAP = 1, SJK_DESC_B = 2, SJK_DESC_N = 3, SJK_DESC_QPOS0 = 4, SJK_DESC_G = 5,
    SJK_DESC_D = 6, SJK_DESC_RECBYTES = 7, SJK_DESC_HKV = 8, SJK_DESC_B_OLD = 9, SJK_DESC_TYPE_K = 10,
    SJK_DESC_TYPE_V = 11, SJK_DESC_BODY_TYPE = 12, SJK_DESC_SINK_TYPE = 13, SJK_DESC_N_ENTRIES = 16
};

/* The commit of sjk_hip_commit with its range [d_desc[SJK_DESC_B_OLD], d_desc[SJK_DESC_B]) read on the device
 * when the kernel runs, launched for n_groups_max groups per layer: the launch does not depend on the range,
 * so a captured HIP graph replays every commit (the reference's ggml_sjkvarn_seal_dyn,
 * INTEGRATION_LLAMACPP.md:48). Groups past the range exit at once. Refused, sealing nothing: a negative
 * entry, an empty or misaligned range, and a range of more than n_groups_max groups (sealing a part would
 * leave records that attention reads unsealed). The range must lie in the views' groups, as for
 * sjk_hip_commit. */
int sjk_hip_commit_dyn(const sjk_hip_view * views, int n_layers, const int32_t * d_desc, int n_groups_max, int iters,
                       void * stream);

/* Causal attention for n_q query rows at positions qpos0.. over [0, min(N, qpos+1)) with sealed end B
 * (sj_kvarn_cuda.cuh:102-135). d_q, d_out: [n_q][n_head][D] fp32, rotated basis; GQA maps query head
 * hq to KV head hq / (n_head / n_head_kv). Any n_q and n_head (a prefill ubatch as well as a decode step):
 * the n_q x n_head / n_head_kv query rows of a KV head are cut into tiles of 16 rows, and a launch takes up to
 * 8 jobs side by side (sharing its workgroups in proportion to their work; each job reads the context). The
 * partial results go to v->work (SJKVARN_ERR_ARG without one). Every layout a layer can have runs
 * on a matrix-core kernel; a hand-built view outside them (another group size, head dimension or record
 * layout) is refused with SJK_ERR_UNSUPPORTED and a message (sjk_last_error), as are the batched, no-alloc and
 * descriptor forms below. */
int sjk_hip_attend(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                   const float * d_q, float scale, float * d_out, void * stream);

/* sjk_hip_attend for callers that cannot allocate device memory (code under stream capture, serving loops
 * that forbid hipMalloc): the same kernels and results, with v->work ignored and the partial results in a
 * static device array of 16 MiB per device, held until the process ends. Views whose workspace would be larger
 * (sjk_hip_workspace_bytes > 16 MiB) are refused with SJKVARN_ERR_CAPACITY (sjk_last_error says why). All
 * calls on one device share the array: calls that overlap on a device (two streams, two threads) race. No
 * counterpart in the reference; it is for callers that cannot allocate. */
int sjk_hip_attend_noalloc(const sjk_hip_view * v, uint32_t B, uint32_t N, uint32_t qpos0, int n_q, int n_head,
                           const float * d_q, float scale, float * d_out, void * stream);

/* sjk_hip_attend with B, N and qpos0 read from the device descriptor d_desc (SJK_DESC_B, SJK_DESC_N,
 * SJK_DESC_QPOS0) when the kernels run, on a launch shape that does not depend on them, so a captured HIP
 * graph replays every decode step (the reference's region-aware flash_attn_ext,
 * ggml_flash_attn_ext_set_sjkvarn, INTEGRATION_LLAMACPP.md:49; n_max plays its n_kv_pad: the positions the
 * view's buffers hold). Every layout sjk_hip_attend takes (D = 128 or 256; every scalar body and the 3/3, 3/2,
 * 2/2 trellis bodies). Results equal sjk_hip_attend's bit for bit. A descriptor
 * the view cannot hold (a negative entry, B misaligned or past N, N past n_max, a tail longer than the ring)
 * writes NaN rows. The call is planned on the device from the descriptor: a 16-row call of the trellis and other
 * scalar bodies in its workgroups, a 4/4 call and any call of more than 16 rows per KV head by a one-workgroup
 * plan kernel that writes the launch's job table into v->work. The table and the partial results live in v->work,
 * which the layer allocated when it was created, so a capture sees no allocation. Any number of query rows per
 * KV head (n_q x n_head / n_head_kv): as in sjk_hip_attend, 16-row tiles, up to 8 a launch, shared out by the
 * same arithmetic; a launch and its combine per 8 tiles, in stream order, all on the one stream a capture
 * records. */
int sjk_hip_attend_dyn(const sjk_hip_view * v, const int32_t * d_desc, uint32_t n_max, int n_q, int n_head,
                       const float * d_q, float scale, float * d_out, void * stream);

/* Batched attention: n_jobs independent calls (each a layer view with its B, N, qpos0, d_q, d_out as in
 * sjk_hip_attend) that share n_q, n_head and scale, e.g. one layer of every sequence of a decode
 * batch. Jobs of one record layout, KV head count and staging type run in one launch (8 per launch);
 * others run one call each. No counterpart in the reference (whose attention is one row and head per
 * call, sj_kvarn.h:1535-1564); each job's result equals its sjk_hip_attend result. */
typedef struct sjk_hip_attend_job {
    sjk_hip_view  v;
    uint32_t      B, N, qpos0;
    const float * d_q;
    float       * d_out;
} sjk_hip_attend_job;
int sjk_hip_attend_batch(const sjk_hip_attend_job * jobs, int n_jobs, int n_q, int n_head, float scale, void * stream);

/* Batched append: n_jobs independent sjk_hip_layer_store calls of n_pos positions each (job = view,
 * pos0, d_k, d_v) in one launch (16 per launch). No counterpart in the reference. */
typedef struct sjk_hip_store_job {
    sjk_hip_view  v;
    uint32_t      pos0;
    const float * d_k;
    const float * d_v;
} sjk_hip_store_job;
int sjk_hip_store_batch(const sjk_hip_store_job * jobs, int n_jobs, uint32_t n_pos, int rotate, void * stream);

/* K and V rows (fp32, rotated) of positions pos0 .. pos0+n_pos-1 of KV head h with sealed end B:
 * d_k, d_v [n_pos][D] (the region resolver of sj_kvarn_layer_kv_row, sj_kvarn.h:1516-1533, and of
 * sj_kvarn_cuda_kv_row, sj_kvarn_cuda.cuh:82-100) */
int sjk_hip_kv_rows(const sjk_hip_view * v, uint32_t B, uint32_t pos0, uint32_t n_pos, int h, float * d_k, float * d_v,
                    void * stream);

/* scores[t] = dot(q, K[t]) and acc[d] += sum_t w[t] V[t,d] for the first n tokens of one device record,
 * sequential fp32 sums as in the reference (sj_kvarn.h:1288-1311) */
int sjk_hip_record_scores(const sj_kvarn_layout * l, const uint8_t * d_rec, const float * d_q, int n, float * d_scores,
                          void * stream);
int sjk_hip_record_accum_v(const sj_kvarn_layout * l, const uint8_t * d_rec, const float * d_w, int n, float * d_acc,
                           void * stream);

/* Device twins of sj_kvarn_seq_store (sj_kvarn.h:407, 1779-1792) and sj_kvarn_seq_attend_row
 * (sj_kvarn.h:414, 1806-1809), one layer il per call: sjk_hip_seq_store appends n_pos positions
 * pos0.. (pos0 <= the sequence's position count) to layer il as sjk_hip_layer_store does and extends
 * the position count; sjk_hip_seq_attend is sjk_hip_attend over layer il with the sequence's sealed
 * end and position count. SJKVARN_ERR_ARG for a bad layer index or a gap before pos0. */
int sjk_hip_seq_store(sj_kvarn_seq * s, int il, uint32_t pos0, uint32_t n_pos, const float * d_k, const float * d_v,
                      int rotate, void * stream);
int sjk_hip_seq_attend(const sj_kvarn_seq * s, int il, uint32_t qpos0, int n_q, int n_head, const float * d_q,
                       float scale, float * d_out, void * stream);

/* The same for layer il of several sequences in one launch each (a decode batch): job k appends n_pos
 * positions from pos0 to seq (sjk_hip_seq_store_batch, d_k / d_v) or runs the n_q query rows at
 * positions pos0.. over it (sjk_hip_seq_attend_batch, d_q / d_out; pos0 + n_q <= the position count). */
typedef struct sjk_hip_seq_job {
    sj_kvarn_seq * seq;
    uint32_t       pos0;
    const float  * d_k;
    const float  * d_v;
    const float  * d_q;
    float        * d_out;
} sjk_hip_seq_job;
int sjk_hip_seq_store_batch(const sjk_hip_seq_job * jobs, int n_jobs, int il, uint32_t n_pos, int rotate, void * stream);

/* Stream-ordered twins of sj_kvarn_seq_begin_ubatch and sj_kvarn_seq_idle (sj_kvarn.h:408-410, 1760-1777): the
 * same policy step and commit, with the seal of [B, B_pending) (every layer, one launch per 64 layers) and the
 * copy of the new block-table entries enqueued on `stream` after what the caller enqueued there before (its
 * stores of earlier positions), and no wait: work the caller enqueues on `stream` afterwards sees the new records.
 * The reference's seal reads only positions below pos0 and may run on a side stream (README.md:351-352): an engine
 * that stores on another stream orders the two itself. A failed launch returns its status with the policy as it
 * was. No counterpart in the reference's C API. */
int sjk_hip_seq_begin_ubatch(sj_kvarn_seq * s, uint32_t pos0, uint32_t n_tokens, void * stream);
int sjk_hip_seq_idle(sj_kvarn_seq * s, uint32_t keep_recent, void * stream);

/* Asynchronous state save and restore (README.md:609 plans "device-to-host copies overlapped with decoding"; no
 * counterpart in the reference's C API). The stream bytes are those of sj_kvarn_seq_state_write / _read.
 *   _write_begin: the checks and header of sj_kvarn_seq_state_write; the sequence's device pieces (sink, records,
 *     ring rows of every layer) are gathered into a device snapshot by one launch before it returns, so the caller
 *     may store into, commit and attend the sequence right away; a host thread then copies the snapshot to dst
 *     (pinned chunks on a stream of the sequence's own) and appends the checksum. dst stays valid until _finish.
 *   _read_begin: the header checks of sj_kvarn_seq_state_read (all but the checksum); a host thread checks the
 *     checksum and uploads the payload into the device snapshot. The sequence is left as it was; the caller does
 *     not use it until _finish, which checks the pool again, resets the sequence and scatters the snapshot into
 *     it with one launch (a rejected stream leaves the sequence unchanged; a device failure in the scatter leaves
 *     it reset, as sj_kvarn_seq_state_read).
 *   _poll: 1 when no transfer is in flight or it has ended, 0 while it runs (never blocks).
 *   _finish: waits for the transfer and returns its status (*written: the stream bytes of a save).
 * One transfer per sequence at a time: state calls on a sequence with one in flight return SJKVARN_ERR_PENDING;
 * sj_kvarn_seq_free waits for it. The snapshot (one stream payload of device memory) is kept with the sequence. */
int sjk_hip_seq_state_write_begin(const sj_kvarn_seq * s, void * dst, size_t dst_size);
int sjk_hip_seq_state_read_begin(sj_kvarn_seq * s, const void * src, size_t size);
int sjk_hip_seq_state_poll(const sj_kvarn_seq * s);
int sjk_hip_seq_state_finish(sj_kvarn_seq * s, size_t * written);
int sjk_hip_seq_attend_batch(const sjk_hip_seq_job * jobs, int n_jobs, int il, int n_q, int n_head, float scale,
                             void * stream);

/* The log-domain scale update of the seal's variance balance, element-wise over device arrays: with
 * s = clamp(d_sd[i], 1e-3, 1e3), d_acc[i] = clamp(d_acc[i] + log((double) s), -0.3, 10) and d_scale[i] =
 * (float) exp(d_acc[i]) (sj_kvarn.h:1000-1002, 1006-1008). It is the seal's own device code, exported so that
 * the device's double log / exp can be compared with the host libm the reference calls. */
int sjk_hip_balance_step(const float * d_sd, double * d_acc, float * d_scale, int n, void * stream);

/* device view of a layer created by sj_kvarn_layer_init / sj_kvarn_seq_init (pool mode: the view
 * carries the sequence's device copy of its block table) */
sjk_hip_view sjk_layer_view(const sj_kvarn_layer * L);

/* last HIP error text seen by the library (for SJK_ERR_DEVICE) */
const char * sjk_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* SJK_H */
