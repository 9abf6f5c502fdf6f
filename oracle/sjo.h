/* sjo.h - CPU oracle for the SJ-KVaRN codec hot path (TEST INFRASTRUCTURE ONLY).
 *
 * A from-scratch C99 restatement of the behaviour of the reference library sj_kvarn.h
 * (JakeATX/sj-kvarn-codec). It exists to check the HIP implementation: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the checker or
 * as the CPU baseline. The product library never links or calls it.
 *
 * Every function cites the reference lines whose results it reproduces. Parity pins:
 *   fp16 conversion       exhaustive over all 2^32 floats against the compiled reference, and
 *                         every half round-trips (tests/test_oracle_fp16.py)
 *   seal / decode / tq6   the 21 FNV-1a vectors of tests/expected_vectors.txt, held as fixtures
 *                         under tests/golden/ (tests/test_oracle_vectors.py)
 *   policy                fuzz against an independent Python transcription (tests/test_oracle_policy.py)
 *   layer / seq / state   the 5 state-stream hashes of tests/expected_state.txt
 *   attention             a float64 softmax over the same decoded rows (tolerance, not bits)
 *   everything            against oracle/_ref (the reference compiled from its own header) on
 *                         seeded inputs at the BASELINE shapes
 *
 * Numerics: build with -std=c99 -ffp-contract=off and without -ffast-math on an SSE2/AArch64
 * target (FLT_EVAL_METHOD 0): every + - * / below then rounds once, as the reference's volatile
 * helpers force (sj_kvarn.h:647-677).
 */
#ifndef SJO_H
#define SJO_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SJO_BODY_SCALAR = 0, SJO_BODY_TRELLIS = 1, SJO_BODY_AUTO = 2 };
enum { SJO_STAGING_TQ6 = 0, SJO_STAGING_F16 = 1 };
enum { SJO_SINK_F16 = 0, SJO_SINK_INHERIT = 1 };

#define SJO_QK          128   /* values per tq6_0 block */
#define SJO_TQ6_BYTES   98
#define SJO_TSEQ        128   /* trellis sequence length */
#define SJO_THIST       6     /* trellis history bits */
#define SJO_NSTATE      64
#define SJO_NO_POS      UINT32_MAX
#define SJO_NO_BLOCK    UINT32_MAX
#define SJO_STATE_HDR   128

/* same field order as sj_kvarn_layout (sj_kvarn.h:170-175): it is the record-layout ABI */
typedef struct sjo_layout {
    int D, G, bits_k, bits_v, body;
    uint32_t k_payload, v_payload, k_scale, k_zero, k_tok, v_ch, v_scale, v_zero, bytes;
} sjo_layout;

typedef struct sjo_policy {
    uint32_t sink, tail, tail_max, group, flush_chunk;
    uint32_t B, B_prev, B_pending;
    int draining;
} sjo_policy;

typedef struct sjo_config {
    int head_dim, n_head_kv, group, bits_k, bits_v, body, iters, staging, sink_type;
    uint32_t sink, tail, tail_max, flush_chunk, n_ubatch, n_ctx;
} sjo_config;

typedef struct sjo_layer {
    sjo_config cfg;
    sjo_layout lay;
    uint32_t cap, n_groups;
    size_t stage_bytes;
    uint8_t *ring, *sink, *body;
    void *work;
    uint16_t *kstage, *vstage;
    const uint32_t *blocks;
    int owns_body;
} sjo_layer;

typedef struct sjo_pool {
    sjo_config cfg;
    sjo_layout lay;
    int n_layers;
    uint32_t n_blocks;
    uint8_t *body;
    uint32_t *free_ids;
    uint32_t n_free;
} sjo_pool;

typedef struct sjo_seq {
    sjo_config cfg;
    int n_layers;
    sjo_layer *layers;
    sjo_policy pol;
    uint32_t n;
    sjo_pool *pool;
    uint32_t *blocks;
} sjo_seq;

typedef struct sjo_state_info {
    uint32_t state_version, format_version;
    sjo_config cfg;
    uint32_t rotation, rotation_n;
    uint64_t codebook_id;
    int n_layers;
    uint32_t n, B, B_prev, draining;
    size_t total_bytes;
} sjo_state_info;

/* fp16 (sj_kvarn.h:693-731) */
uint16_t sjo_f32_to_f16(float f);
float    sjo_f16_to_f32(uint16_t h);

/* rotation (sj_kvarn.h:735-759) */
void sjo_hadamard(float *x, int n);
void sjo_rotate_heads(float *x, int n_heads, int head_dim);

/* layout (sj_kvarn.h:763-849) */
int      sjo_body_resolve(int body, int bits_k, int bits_v);
int      sjo_layout_init(sjo_layout *l, int D, int G, int bits_k, int bits_v, int body);
size_t   sjo_record_bytes(int D, int G, int bits_k, int bits_v);
uint32_t sjo_code_bit(const sjo_layout *l, int t, int d, int is_v);
int      sjo_k_ch_idx(const sjo_layout *l, int d);
int      sjo_v_ch_idx(const sjo_layout *l, int d);

/* seal / decode (sj_kvarn.h:906-1207) */
size_t sjo_seal_workspace_bytes(const sjo_layout *l);
void   sjo_seal_group(const sjo_layout *l, const uint16_t *K, const uint16_t *V, size_t row_stride, int iters,
                      uint8_t *rec, void *work);
void   sjo_decode_k_row(const sjo_layout *l, const uint8_t *rec, int t, float *out);
void   sjo_decode_v_row(const sjo_layout *l, const uint8_t *rec, int t, float *out);

/* staging (sj_kvarn.h:1211-1284); blocks are 98-byte {u16 norm; u8 qs[64]; u8 qh[32]} */
void   sjo_tq6_quantize_row(const float *x, uint8_t *blocks, int n);
void   sjo_tq6_dequantize_row(const uint8_t *blocks, float *x, int n);
size_t sjo_stage_row_bytes(int staging, int D);
void   sjo_stage_row(int staging, const float *x_rot, void *dst, int D);
void   sjo_unstage_row(int staging, const void *src, float *x_rot, int D);

/* attention helpers (sj_kvarn.h:1288-1311) */
/* the balance's log-domain scale update (sj_kvarn.h:1000-1002) over arrays: acc in place, scale out */
void sjo_balance_step(const float *sd, double *acc, float *scale, size_t n);
void sjo_record_scores(const sjo_layout *l, const uint8_t *rec, const float *q, int n, float *scores);
void sjo_record_accum_v(const sjo_layout *l, const uint8_t *rec, const float *w, int n, float *acc);

/* policy (sj_kvarn.h:1315-1407) */
void     sjo_policy_init(sjo_policy *p, uint32_t sink, uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t flush_chunk);
void     sjo_policy_reset(sjo_policy *p);
uint32_t sjo_policy_begin_ubatch(sjo_policy *p, uint32_t pos0, uint32_t n_tokens);
void     sjo_policy_commit(sjo_policy *p);
uint32_t sjo_policy_idle(sjo_policy *p, uint32_t end, uint32_t keep_recent);
uint32_t sjo_group_floor(uint32_t sink, uint32_t group, uint32_t pos);
uint32_t sjo_policy_trunc_floor(const sjo_policy *p, uint32_t pos);
uint32_t sjo_policy_truncate(sjo_policy *p, uint32_t pos, uint32_t *n_dropped);
uint32_t sjo_ring_capacity(uint32_t tail, uint32_t tail_max, uint32_t group, uint32_t n_ubatch);
uint32_t sjo_ring_slot(uint32_t sink, uint32_t cap, uint32_t pos);

/* per-layer cache (sj_kvarn.h:1411-1603) */
sjo_config sjo_config_default(int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch);
void       sjo_config_default_into(sjo_config *c, int head_dim, int n_head_kv, uint32_t n_ctx, uint32_t n_ubatch);
int        sjo_layer_init(sjo_layer *L, const sjo_config *cfg);
void       sjo_layer_free(sjo_layer *L);
void       sjo_layer_store(sjo_layer *L, uint32_t pos, const float *k_rot, const float *v_rot);
void       sjo_layer_seal(sjo_layer *L, uint32_t B_from, uint32_t B_to);
void       sjo_layer_kv_row(const sjo_layer *L, uint32_t B, uint32_t pos, int h, float *k, float *v);
void       sjo_layer_attend_row(const sjo_layer *L, uint32_t B, uint32_t N, const float *q_rot, int h, uint32_t qpos,
                                float scale, float *out_rot);
uint8_t   *sjo_layer_record(const sjo_layer *L, uint32_t g, int h);
void       sjo_layer_truncate(sjo_layer *L, uint32_t B_old, uint32_t B_new, uint32_t n_old, uint32_t resume);
const char *sjo_strerror(int code);

/* pool / sequence / state (sj_kvarn.h:1645-2034) */
int      sjo_pool_init(sjo_pool *pool, const sjo_config *cfg, int n_layers, uint32_t n_blocks);
void     sjo_pool_free(sjo_pool *pool);
uint32_t sjo_pool_alloc(sjo_pool *pool);
void     sjo_pool_release(sjo_pool *pool, uint32_t id);
int      sjo_seq_init(sjo_seq *s, const sjo_config *cfg, int n_layers, sjo_pool *pool);
void     sjo_seq_free(sjo_seq *s);
void     sjo_seq_reset(sjo_seq *s);
int      sjo_seq_begin_ubatch(sjo_seq *s, uint32_t pos0, uint32_t n_tokens);
void     sjo_seq_store(sjo_seq *s, uint32_t pos, const float *k_rot, const float *v_rot);
int      sjo_seq_idle(sjo_seq *s, uint32_t keep_recent);
uint32_t sjo_seq_truncate(sjo_seq *s, uint32_t pos);
void     sjo_seq_attend_row(const sjo_seq *s, int il, const float *q_rot, int h, uint32_t qpos, float scale, float *out_rot);
size_t   sjo_seq_state_size(const sjo_seq *s);
size_t   sjo_state_size_max(const sjo_config *cfg, int n_layers);
int      sjo_seq_state_write(const sjo_seq *s, void *dst, size_t dst_size, size_t *written);
int      sjo_state_peek(const void *src, size_t size, sjo_state_info *info);
int      sjo_seq_state_read(sjo_seq *s, const void *src, size_t size);

/* ---- test-support generators (integer-only, host-independent) ---- */
uint64_t sjo_fnv1a(const void *p, size_t n, uint64_t h);
#define SJO_FNV0 UINT64_C(1469598103934665603)
/* the reference's vector inputs (tests/vector_inputs.h:8-50): one (group, head) of fp16 K/V rows */
void sjo_vec_fill_group(int D, int G, uint32_t seed, uint16_t *K, uint16_t *V);
void sjo_vec_fill_rows(int rows, int n, float *x);
/* the reference state test's position-addressable rows (tests/test_state.c:33-53) */
float sjo_st_val(uint32_t seed, uint32_t variant, uint32_t pos, uint32_t i, int side);
int   sjo_st_grow(sjo_seq *q, uint32_t seed, uint32_t edit_from, uint32_t edit_variant, uint32_t from, uint32_t to,
                  uint32_t pattern);

#ifdef __cplusplus
}
#endif
#endif
