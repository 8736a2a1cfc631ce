/*
 * kanso_hip.h — C ABI of libkanso_hip.so, the MI355X (gfx950) implementation of
 * kanso-infer's ragged continuous-batching attention path.
 *
 * Every function is `extern "C"`, takes plain pointers and sizes, and returns an
 * int status (KANSO_OK = 0, negative on error). The message of the last error on
 * the calling thread is kanso_last_error(). Shapes the kernels cannot represent are
 * errors, never silent fallbacks (reference: src/metal/paged_attention.rs:34-38).
 *
 * Ownership: the caller owns every buffer named in an argument list (device
 * memory unless stated otherwise). A kanso_ctx owns only its scratch: split-K
 * partials, the attention work list and a device status word. A context is not
 * thread-safe; work is enqueued asynchronously on the caller's stream.
 *
 * Device-side validation: conditions that depend on device-resident data (a
 * context length of 0, a slot outside the pool, a block table too short for a
 * position) cannot be checked on the host without a synchronisation. The kernels
 * clamp so they never read or write out of bounds, record the condition in the
 * context's status word, and kanso_check_device_status() reports it.
 *
 * Reference interfaces replaced (paths relative to the kanso-infer tree):
 *   src/metal/paged_attention.rs:12-22    PagedAttentionParams     -> kanso_paged_attention_params
 *   src/metal/paged_attention.rs:27-32    num_partitions           -> kanso_paged_attention_num_partitions
 *   src/metal/paged_attention.rs:39-81    validate_...params       -> kanso_validate_paged_attention_params
 *   src/metal/paged_attention.rs:193-293  encode_paged_attention_v2-> kanso_paged_attention_v2
 *   src/model.rs:1689-1714 (mixed-batch per-sequence gqa_attention)-> kanso_ragged_paged_attention
 *   src/engine.rs:376-402 + src/model.rs:64-116 (step packing)    -> kanso_pack_step
 *   src/kv_cache/kind.rs:348-374 write_kv_slots                   -> kanso_kv_append
 *   src/kv_cache/kind.rs:379-387 reset_block                      -> kanso_kv_reset_blocks
 *   src/weights.rs:43-45 LinearWeight::forward on Q8_0 / Q4_K     -> kanso_gemv_q8_0 / kanso_gemv_q4_k
 */
#ifndef KANSO_HIP_H
#define KANSO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t, declared opaquely so this header does not need the HIP headers.
 * NULL means the default (null) stream of the current device. */
typedef struct ihipStream_t* kanso_stream_t;

typedef struct kanso_ctx kanso_ctx;

/* Status codes (reference EngineError variants, src/error.rs:4-11, become codes). */
enum {
    KANSO_OK = 0,
    KANSO_E_INVALID_ARG = -1,   /* null pointer, zero where non-zero is required  */
    KANSO_E_INVALID_SHAPE = -2, /* shape outside what the kernels represent       */
    KANSO_E_OUT_OF_BOUNDS = -3, /* index / slot / length outside its buffer       */
    KANSO_E_HIP = -4,           /* a HIP runtime call failed                      */
    KANSO_E_DEVICE_CHECK = -5   /* a device-side validation flag was raised       */
};

/* Bits of the device status word (kanso_check_device_status). */
enum {
    KANSO_DEV_EMPTY_CONTEXT = 1u << 0,    /* context_len == 0 (paged_attention.rs:349-355)   */
    KANSO_DEV_CONTEXT_OVERFLOW = 1u << 1, /* context_len > table capacity (:342-348)         */
    KANSO_DEV_QUERY_OVERFLOW = 1u << 2,   /* query rows > context_len (model.rs:1488-1493)   */
    KANSO_DEV_TABLE_SHORT = 1u << 3,      /* block table shorter than needed (engine.rs:387) */
    KANSO_DEV_SLOT_OOB = 1u << 4,         /* slot >= num_blocks*block_size (kind.rs:130-137) */
    KANSO_DEV_BLOCK_OOB = 1u << 5,        /* physical block id >= num_blocks                 */
    KANSO_DEV_POSITION_OOB = 1u << 6,     /* position beyond the RoPE table                  */
    KANSO_DEV_TOKEN_OOB = 1u << 7,        /* token id >= vocab size                          */
    KANSO_DEV_PARTS_OOB = 1u << 8         /* a row's partition count beyond the partials'    */
                                          /* capacity (a work list missing a row's items)    */
};

/* KV pool element types.
 *   F32:  pool [num_blocks][block_size][num_kv_heads][head_dim] f32
 *         (src/kv_cache/storage.rs:70-76).
 *   INT8: quant [num_blocks][block_size][num_kv_heads][head_dim] i8 and
 *         scales [num_blocks][block_size][num_kv_heads] f32, one scale per token per
 *         KV head (src/kv_cache/quantized_storage.rs:14-21, 452-469).
 *   Q8_0: quant [num_blocks][block_size][num_kv_heads][head_dim] i8 and
 *         scales [num_blocks][block_size][num_kv_heads][head_dim/32] f16 (IEEE
 *         binary16 bits), one scale per 32 elements, quantized with the Q8_0 rule
 *         of src/quant/q8_0.rs:13-32; head_dim must be a multiple of 32.       */
/* KV pool kinds. INT8 and FP8 keep one f32 scale per (token, KV head) and
 * head_dim bytes per row (src/kv_cache/quantized_storage.rs:433-489); FP8 bytes are
 * OCP E4M3FN (bias 7, no infinities, NaN = S.1111.111). Q8_0 keeps one f16 scale
 * per 32 elements (head_dim % 32 == 0). */
enum { KANSO_KV_F32 = 0, KANSO_KV_INT8 = 1, KANSO_KV_Q8_0 = 2, KANSO_KV_FP8 = 3 };

/* Row order inside a pool block (every pool tensor and its scales alike).
 *   TOKEN_MAJOR: [num_blocks][block_size][num_kv_heads][...], the reference's
 *                (src/kv_cache/storage.rs:70-76);
 *   HEAD_MAJOR:  [num_blocks][num_kv_heads][block_size][...]: one (block, KV head)
 *                is block_size contiguous rows, the layout this build's engine
 *                uses (contiguous 4 KB runs per head at head_dim 64, F32). */
enum { KANSO_POOL_TOKEN_MAJOR = 0, KANSO_POOL_HEAD_MAJOR = 1 };

/* Same fields, order and types as PagedAttentionParams (src/metal/paged_attention.rs:12-22). */
typedef struct {
    uint32_t num_seqs;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t block_size;
    uint32_t max_num_blocks_per_seq;
    float scale;
} kanso_paged_attention_params;

/* Parameters of one ragged (mixed prefill + decode) attention call. */
typedef struct {
    uint32_t num_seqs;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t block_size;
    uint32_t max_num_blocks_per_seq; /* row stride of block_tables                 */
    float scale;
    uint32_t total_q;    /* T = cu_seqlens[num_seqs]: query rows in q and out       */
    uint32_t kv_dtype;   /* KANSO_KV_*                                              */
    uint32_t num_blocks; /* physical blocks in the pool (bounds check of table ids) */
    uint32_t max_q_len;  /* upper bound of any sequence's query rows (0 = total_q)  */
    uint32_t pool_layout; /* KANSO_POOL_*                                           */
    uint32_t partition_size; /* split-K partition of decode rows in tokens: 0 = chosen
                                from the shape; else a multiple of 32 in
                                [32, min(992, 62 * block_size)]
                                (kanso_ragged_partition_size picks one)           */
    uint32_t chunk_partition_size; /* split-K partition of the rows of sequences with
                                more than one query row (matrix-core chunk items):
                                0 = max(partition, 512, within 62 blocks); else a
                                multiple of 32 in [32, min(992, 62 * block_size)]
                                (kanso_ragged_chunk_partition_size picks one)     */
} kanso_ragged_attention_params;

/* One planned sequence of a step, as Engine::step plans it (src/engine.rs:221-226). */
typedef struct {
    uint32_t start_pos;    /* position of the first query token                    */
    uint32_t q_len;        /* tokens this step: 1 for decode, chunk_len for prefill */
    uint32_t table_offset; /* first entry of this sequence's table in table_arena   */
    uint32_t table_len;    /* entries of the table                                  */
    uint32_t token_offset; /* token at position pos is token_arena[token_offset + pos]
                              (32-bit unsigned arithmetic)                           */
} kanso_seq_plan;

/* Device outputs of kanso_pack_step (all caller-owned device buffers). */
typedef struct {
    int32_t* cu_seqlens;    /* [S+1] prefix sums of q_len                            */
    int32_t* seq_of_query;  /* [T]   sequence index of every query row                */
    int32_t* positions;     /* [T]   start_pos + i                                    */
    int64_t* slot_mapping;  /* [T]   table[pos / bs] * bs + pos % bs                  */
    uint32_t* tokens;       /* [T]   token_arena[token_offset + pos]                  */
    uint32_t* block_tables; /* [S * max_blocks] padded by repeating table[needed-1]   */
    uint32_t* context_lens; /* [S]   start_pos + q_len                                */
} kanso_packed_step;

const char* kanso_last_error(void);

/* Context on HIP device `device`. */
int kanso_create(int device, kanso_ctx** out);
int kanso_destroy(kanso_ctx* ctx);

/* Synchronises `stream`, reads and clears the device status word. Returns
 * KANSO_E_DEVICE_CHECK (and the bits in *flags) when any was raised. */
int kanso_check_device_status(kanso_ctx* ctx, kanso_stream_t stream, uint32_t* flags);

/* ceil(max_num_blocks_per_seq * block_size / 256), at least 1
 * (src/metal/paged_attention.rs:27-32). */
uint32_t kanso_paged_attention_num_partitions(const kanso_paged_attention_params* p);

/* Host-side shape validation (src/metal/paged_attention.rs:39-81). This build's
 * limits: GQA group <= 8, head_dim a power of two in [4, 256]. */
int kanso_validate_paged_attention_params(const kanso_paged_attention_params* p);

/* Decode attention over an F32 pool: q [num_seqs][num_heads][head_dim], one query
 * per sequence attending its context_lens[s] tokens through block_tables
 * [num_seqs][max_num_blocks_per_seq]; out [num_seqs][num_heads][head_dim].
 * Replaces encode_paged_attention_v2 (src/metal/paged_attention.rs:193-203). */
int kanso_paged_attention_v2(kanso_ctx* ctx, const kanso_paged_attention_params* p,
                             const float* q, const float* k_cache, const float* v_cache,
                             const uint32_t* block_tables, const uint32_t* context_lens,
                             float* out, kanso_stream_t stream);

/* Ragged attention over a mixed batch. Sequence s owns query rows
 * cu_seqlens[s]..cu_seqlens[s+1] (q_len rows); row i sits at position
 * context_lens[s] - q_len + i and attends keys 0..=that position (the offset causal
 * mask of src/model.rs:1510-1527; a decode row attends its whole context).
 * q and out are [total_q][num_heads][head_dim] f32. k_scales/v_scales are unused
 * for KANSO_KV_F32. Query head h reads KV head h / (num_heads/num_kv_heads).
 * cu_seqlens may be null for a decode batch (total_q == num_seqs, max_q_len 1):
 * one row per sequence. */
/* The split-K partition for kanso_ragged_paged_attention's partition_size, from the
 * step's host-side query and context lengths (num_seqs entries each), which the
 * caller that planned the step holds (Engine::step's query_lens / context_lens,
 * src/engine.rs:376-402): the smallest multiple of 32 (<= 512) for which every
 * decode item (row x KV head x partition) gets a resident wave in one pass, with
 * chunk items on their own partition of at least 512 keys. No counterpart in the
 * reference (its Metal kernel uses a fixed PARTITION_SIZE of 256). Returns 0 (=
 * let the library choose) for unusable arguments. Host-only; launches nothing. */
uint32_t kanso_ragged_partition_size(const kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                     const uint32_t* q_lens, const uint32_t* context_lens);

/* The chunk partition for chunk_partition_size, from the same host-side lengths.
 * A batch with a decode row returns 0 (chunk items keep long partitions, so they
 * hold few of the CU slots the decode waves stream in). A batch of multi-row
 * sequences only (prefill chunks, speculative verify rows) returns the smallest
 * multiple of 32 (at least 64) for which the chunk items fit the resident
 * workgroups in one pass: shorter items, run side by side. No counterpart in the
 * reference. Returns 0 for unusable arguments. Host-only; launches nothing. */
uint32_t kanso_ragged_chunk_partition_size(const kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                           const uint32_t* q_lens, const uint32_t* context_lens);

int kanso_ragged_paged_attention(kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                 const float* q, const void* k_pool, const void* v_pool,
                                 const void* k_scales, const void* v_scales,
                                 const uint32_t* block_tables, const int32_t* cu_seqlens,
                                 const uint32_t* context_lens, float* out,
                                 kanso_stream_t stream);

/* Work list of a planned batch. The caller that planned the step holds its query
 * lengths, context lengths and block tables on the host (Engine::step's
 * query_lens / context_lens / block tables, src/engine.rs:376-402); from them
 * kanso_ragged_build_work writes items of KANSO_RAGGED_WORK_ITEM_WORDS u32: first one
 * per (row, partition) of every row outside the matrix-core chunk path (the
 * partition's physical block ids, then row, first key, end key, the row's key
 * count), then one per (64-row block, chunk partition) of the sequences on that path
 * (block ids, then first row, rows, key position of the first row, partition).
 * kanso_ragged_paged_attention_work takes that list (uploaded to the device) instead
 * of deriving the items from the sequence and block tables: a wave's first load is
 * its item, its second its keys. Results are bit-identical to
 * kanso_ragged_paged_attention's. p->partition_size must be set
 * (kanso_ragged_partition_size); partitions of at most 60 blocks; F32 / INT8 / Q8_0
 * pools, token-major layout; every row must have a key. kanso_ragged_work_items
 * returns the item count (and the chunk items among them), 0 when the batch cannot
 * take a list (then call kanso_ragged_paged_attention). No counterpart in the
 * reference (the Metal kernel derives its work from the grid). block_tables is the
 * host copy of the [num_seqs][max_num_blocks_per_seq] table the attention call
 * reads. The first two are host-only and launch nothing. The list must be the one
 * kanso_ragged_build_work wrote for these lengths: a list that leaves out a row's
 * items leaves that row's output unwritten, and when its stale partition count
 * exceeds the call's partials the merge skips the row and raises
 * KANSO_DEV_PARTS_OOB. */
#define KANSO_RAGGED_WORK_ITEM_WORDS 64u
uint32_t kanso_ragged_work_items(const kanso_ragged_attention_params* p, const uint32_t* q_lens,
                                 const uint32_t* context_lens, uint32_t* n_chunk_items);
int kanso_ragged_build_work(const kanso_ragged_attention_params* p, const uint32_t* q_lens,
                            const uint32_t* context_lens, const uint32_t* block_tables, uint32_t* work,
                            uint32_t n_items);
int kanso_ragged_paged_attention_work(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q,
                                      const void* k_pool, const void* v_pool, const void* k_scales,
                                      const void* v_scales, const uint32_t* block_tables,
                                      const int32_t* cu_seqlens, const uint32_t* context_lens, float* out,
                                      const uint32_t* work, uint32_t n_items, uint32_t n_chunk_items,
                                      kanso_stream_t stream);

/* kanso_ragged_paged_attention without any allocation: the same kernels, with
 * their split-K partials, statistics and per-row partition counts in a fixed
 * 64 MiB device array that each GPU holds for the life of the process (its
 * address is resolved at kanso_create), and no profiling events. A call whose
 * scratch (rows x heads x partitions x (head_dim + 2) x 4 B, plus 4 B per row)
 * exceeds 64 MiB is rejected with KANSO_E_INVALID_SHAPE. Every call on one GPU
 * shares that array: calls that overlap on one GPU (several streams or threads)
 * race, and must be serialised by the caller. Nothing in the array needs to start
 * at zero (each call writes before it reads). No counterpart in the reference:
 * for callers that cannot allocate (code under graph capture, serving loops that
 * forbid hipMalloc). */
int kanso_ragged_paged_attention_noalloc(kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                         const float* q, const void* k_pool, const void* v_pool,
                                         const void* k_scales, const void* v_scales,
                                         const uint32_t* block_tables, const int32_t* cu_seqlens,
                                         const uint32_t* context_lens, float* out,
                                         kanso_stream_t stream);

/* Packs one scheduler step on the device (src/engine.rs:376-402 and the padding
 * rule of src/model.rs:64-116). `plan` is a device array of num_seqs entries in plan
 * order; total_q = sum of q_len and max_blocks = max_s ceil((start+q_len)/bs) (at
 * least 1) are computed by the caller from the same plan and size the outputs. */
int kanso_pack_step(kanso_ctx* ctx, const kanso_seq_plan* plan, uint32_t num_seqs,
                    const uint32_t* token_arena, const uint32_t* table_arena,
                    uint32_t block_size, uint32_t max_blocks, uint32_t total_q,
                    const kanso_packed_step* out, kanso_stream_t stream);

/* Writes num_tokens rows of K and V ([num_tokens][num_kv_heads][head_dim] f32) into
 * pool row slot_mapping[t] (slot = block * block_size + offset), quantizing on the
 * fly for INT8 / Q8_0 (src/kv_cache/kind.rs:348-374, quantized_storage.rs:143-204). */
int kanso_kv_append(kanso_ctx* ctx, uint32_t kv_dtype, const float* k, const float* v,
                    const int64_t* slot_mapping, uint32_t num_tokens, uint32_t num_blocks,
                    uint32_t block_size, uint32_t num_kv_heads, uint32_t head_dim,
                    void* k_pool, void* v_pool, void* k_scales, void* v_scales,
                    kanso_stream_t stream);

/* Erases num_reset physical blocks (device array `blocks`) of one pool: F32 and
 * quant bytes to 0, INT8 scales to 1.0, Q8_0 scales to 0 (src/kv_cache/storage.rs:
 * 152-176, quantized_storage.rs:35-40). */
int kanso_kv_reset_blocks(kanso_ctx* ctx, uint32_t kv_dtype, const uint32_t* blocks,
                          uint32_t num_reset, uint32_t num_blocks, uint32_t block_size,
                          uint32_t num_kv_heads, uint32_t head_dim, void* k_pool,
                          void* v_pool, void* k_scales, void* v_scales,
                          kanso_stream_t stream);

/* y[b][out] = sum_i W[out][i] * x[b][i] with W in GGUF block_q8_0 layout
 * ([out][in/32] blocks of {f16 d; i8 qs[32]}, 34 B); in % 32 == 0, batch >= 1.
 * Dequantization semantics of src/quant/q8_0.rs:35-39 / 51-93; bf16 matrix cores
 * with x split into bf16 hi + lo, f32 accumulation. */
int kanso_gemv_q8_0(kanso_ctx* ctx, const void* w, const float* x, float* y,
                    uint32_t out_features, uint32_t in_features, uint32_t batch,
                    kanso_stream_t stream);

/* Same with W in GGUF block_q4_K layout ([out][in/256] blocks of {f16 d; f16 dmin;
 * u8 scales[12]; u8 qs[128]}, 144 B); in % 256 == 0, batch >= 1, w and x 16-byte
 * aligned. Dequantization semantics of src/quant/q4_k.rs:16-55 (d1 q - m1 per
 * 32-element sub-block), on the same matrix-core kernel as kanso_gemv_q8_0. */
int kanso_gemv_q4_k(kanso_ctx* ctx, const void* w, const float* x, float* y,
                    uint32_t out_features, uint32_t in_features, uint32_t batch,
                    kanso_stream_t stream);

/* ---- packed Q8_0 weights and the decoder-layer operations ----------------
 *
 * Packed Q8_0: the GGUF block_q8_0 bytes re-laid for the matrix cores, one 544 B
 * tile per (16-row group, 32-column block): qs[4][16][8] (row r's bytes 8j..8j+7
 * of the block at offset 128 j + 8 r) followed by d[16] (f16). The group count is
 * rounded up to an even number (pairs of groups); rows past the matrix are zero.
 * No reference counterpart: it is this build's device layout of the weights that
 * LinearWeight::forward (src/weights.rs:43-45) reads as GGUF blocks. */

/* Bytes of a packed matrix of `rows` rows (groups rounded up to a multiple of 2). */
size_t kanso_q8_0_packed_bytes(uint32_t rows, uint32_t in_features);

/* Re-lays a GGUF Q8_0 matrix [rows][in/32] into packed groups: source group g
 * (rows 16g..16g+15) becomes destination group g * group_stride + group_offset.
 * Stride 1 / offsets concatenate matrices (Q, K, V); stride 2 interleaves two
 * (gate at offset 0, up at offset 1). Destination groups not written keep their
 * bytes, so the caller zero-fills the buffer first. */
int kanso_q8_0_pack(kanso_ctx* ctx, const void* gguf, uint32_t rows, uint32_t in_features,
                    void* packed, uint32_t group_stride, uint32_t group_offset,
                    kanso_stream_t stream);

/* y[t][out] = W x[t] over a packed matrix (same arithmetic as kanso_gemv_q8_0). */
int kanso_gemm_q8_0(kanso_ctx* ctx, const void* packed, const float* x, float* y,
                    uint32_t out_features, uint32_t in_features, uint32_t num_tokens,
                    kanso_stream_t stream);

/* y[t][out] += W x[t]: the O and down projections with the residual add
 * (src/model.rs:1716-1721: hidden = hidden + linear(...)). */
int kanso_gemm_q8_0_residual(kanso_ctx* ctx, const void* packed, const float* x, float* y,
                             uint32_t out_features, uint32_t in_features,
                             uint32_t num_tokens, kanso_stream_t stream);

/* out[t][:] = row tokens[t] of a packed Q8_0 embedding table, dequantized
 * (Model::embed, src/model.rs:425-431; BlockQ8_0::dequantize, src/quant/q8_0.rs:35-39).
 * Ids >= vocab raise KANSO_DEV_TOKEN_OOB and read row 0. */
int kanso_embed_q8_0(kanso_ctx* ctx, const void* packed_table, uint32_t vocab, uint32_t hidden,
                     const uint32_t* tokens, uint32_t num_tokens, float* out,
                     kanso_stream_t stream);

typedef struct {
    uint32_t num_tokens;
    uint32_t hidden;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;   /* 64 */
    uint32_t max_pos;    /* rows of the cos / sin tables                          */
    float eps;           /* RMSNorm epsilon                                        */
    uint32_t num_blocks; /* pool geometry, for the slot bounds check               */
    uint32_t block_size;
} kanso_qkv_params;

/* One layer's attention prologue for num_tokens rows of x [T][hidden]:
 * RMSNorm(x) * norm_w (src/model.rs:653-659), the Q/K/V projections of the packed
 * row-concatenation [Wq; Wk; Wv] (project_qkv, :437-475), rotate-half RoPE on Q
 * and K with cos/sin rows positions[t] of [max_pos][head_dim/2] tables
 * (rope_apply, :720-737), Q to q_out [T][num_heads][64], K and V written to F32
 * pool row slot_mapping[t] (write_kv_slots, src/kv_cache/storage.rs:219-254). */
int kanso_qkv_rope_append(kanso_ctx* ctx, const kanso_qkv_params* p, const void* packed_qkv,
                          const float* x, const float* norm_w, const int32_t* positions,
                          const int64_t* slot_mapping, const float* cos_table,
                          const float* sin_table, float* q_out, float* k_pool, float* v_pool,
                          kanso_stream_t stream);

/* kanso_qkv_rope_append for a 1-byte pool (kv_dtype KANSO_KV_INT8, KANSO_KV_FP8 or
 * KANSO_KV_Q8_0, the layouts of kanso_kv_append): each token's K and V rows are
 * rotated, quantized (quantize_head_slice, src/kv_cache/quantized_storage.rs:452-486;
 * BlockQ8_0::from_f32_slice, src/quant/q8_0.rs:13-32) and written with their scales
 * to pool row slot_mapping[t] in the product's epilogue, the bytes
 * kanso_qkv_rope_append into F32 rows followed by kanso_kv_append would write
 * (write_kv_slots of the quantized storage, src/kv_cache/kind.rs:348-374), in one
 * kernel. */
int kanso_qkv_rope_append_quant(kanso_ctx* ctx, const kanso_qkv_params* p, const void* packed_qkv,
                                const float* x, const float* norm_w, const int32_t* positions,
                                const int64_t* slot_mapping, const float* cos_table,
                                const float* sin_table, float* q_out, uint32_t kv_dtype, void* k_pool,
                                void* v_pool, void* k_scales, void* v_scales, kanso_stream_t stream);

/* h[t][j] = silu(g) * u with g, u the gate / up projections of RMSNorm(x[t]) *
 * norm_w (forward_mlp_block, src/model.rs:367-380); packed_gate_up interleaves the
 * gate and up groups (kanso_q8_0_pack stride 2). intermediate % 16 == 0. */
int kanso_gate_up_swiglu(kanso_ctx* ctx, const void* packed_gate_up, const float* x,
                         const float* norm_w, float eps, uint32_t num_tokens, uint32_t hidden,
                         uint32_t intermediate, float* h, kanso_stream_t stream);

/* Final RMSNorm (norm_w may be NULL to skip it) of rows x[rows[i]] (rows NULL:
 * x[i]), the lm_head projection and greedy_token (src/sampler.rs:7-17: the first
 * maximum wins; NaN never wins): tokens[i] = argmax. logits [num_rows][vocab] is
 * written when non-NULL (src/model.rs:1729-1738). */
int kanso_lm_head_argmax(kanso_ctx* ctx, const void* packed, const float* x, const int32_t* rows,
                         const float* norm_w, float eps, uint32_t num_rows, uint32_t hidden,
                         uint32_t vocab, float* logits, uint32_t* tokens, kanso_stream_t stream);

/* Q8_0 quantization of n f32 values (n % 32 == 0) into GGUF blocks, on the device:
 * per 32 values d = amax / 127, id = d != 0 ? 1 / d : 0, q = round(x * id) clamped
 * to [-128, 127] (BlockQ8_0::from_f32_slice, src/quant/q8_0.rs:13-32), d stored as
 * f16 (round to nearest even). Bit-exact with the CPU rule. */
int kanso_quantize_q8_0(kanso_ctx* ctx, const float* x, uint64_t n, void* gguf_out,
                        kanso_stream_t stream);

/* ---- the decoder model and the continuous-batching engine ----------------
 *
 * kanso_model: a llama decoder (RMSNorm, rotate-half RoPE, GQA attention, SwiGLU
 * MLP) with packed Q8_0 projections and an F32 paged KV pool, all device
 * resident — the Model of src/model.rs behind forward_batch (:1360-1380).
 * kanso_engine: Engine::step (src/engine.rs:213-505) in C++ driving it. */

typedef struct kanso_model kanso_model;
typedef struct kanso_engine kanso_engine;

typedef struct {
    uint32_t hidden;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;      /* 64 */
    uint32_t num_layers;
    uint32_t intermediate;  /* multiple of 32 */
    uint32_t vocab;
    float eps;              /* RMSNorm epsilon (1e-5)                            */
    float rope_theta;       /* 10000                                             */
    uint32_t max_position;  /* RoPE table rows (positions 0 .. max_position-1)   */
    uint32_t tied_embeddings; /* 1: lm_head is the embedding table              */
    /* Granite multipliers (src/weights.rs:395-406, applied as src/model.rs:424-430,
     * 739-760); 0 = absent (llama: identity, attention 1/sqrt(head_dim)). */
    float embedding_scale;  /* embedding rows x embedding_scale                 */
    float attention_scale;  /* replaces 1/sqrt(head_dim) when non-zero          */
    float residual_scale;   /* attention / FFN outputs x residual_scale before the add */
    float logit_scale;      /* logits x (1 / logit_scale)                       */
} kanso_model_config;

/* Weight kinds of kanso_model_set_weight. Matrices are GGUF Q8_0 bytes [rows][in/32]
 * x 34 B; norms are f32 [hidden]. Per-layer kinds take the layer index. */
enum {
    KANSO_W_EMBED = 0,      /* [vocab][hidden]                 */
    KANSO_W_LM_HEAD = 1,    /* [vocab][hidden] (untied only)   */
    KANSO_W_FINAL_NORM = 2,
    KANSO_W_ATTN_NORM = 3,
    KANSO_W_FFN_NORM = 4,
    KANSO_W_Q = 5,          /* [heads*64][hidden]              */
    KANSO_W_K = 6,          /* [kv_heads*64][hidden]           */
    KANSO_W_V = 7,
    KANSO_W_O = 8,          /* [hidden][heads*64]              */
    KANSO_W_GATE = 9,       /* [intermediate][hidden]          */
    KANSO_W_UP = 10,
    KANSO_W_DOWN = 11       /* [hidden][intermediate]          */
};

int kanso_model_create(kanso_ctx* ctx, const kanso_model_config* cfg, kanso_model** out);
int kanso_model_destroy(kanso_model* model);

/* Uploads one weight from host memory (bytes must match the kind's size) and
 * re-lays matrices into the packed layout. */
int kanso_model_set_weight(kanso_model* model, uint32_t kind, uint32_t layer,
                           const void* host_data, size_t bytes);

/* Uploads one projection matrix in GGUF Q4_K blocks ([rows][in/256] x 144 B;
 * in a multiple of 256), kept in that format and multiplied by the Q4_K loader of
 * the product kernels (the reference keeps any GGUF block type as a QMatMul,
 * src/weights.rs:33-39). Kinds: Q, K, V, O, GATE, UP, DOWN. A layer's Q, K and V
 * (and its gate and up) run in one fused product, so they must all be Q4_K or
 * all Q8_0: a forward over a layer with a mix is refused. */
int kanso_model_set_weight_q4_k(kanso_model* model, uint32_t kind, uint32_t layer,
                                const void* host_data, size_t bytes);

/* Random-init weights generated on the device (create_mock_*, src/model.rs:520-651,
 * with SmolLM2's std of 0.02 in place of N(0,1)): matrix j (embedding 1, untied
 * lm_head 2, then per layer Q, K, V, O, gate, up, down) draws element i from
 * splitmix64(seed_j ^ (i * 0xd1342543de82ef95)), seed_j = seed * 0x100000001b3 +
 * j * 0x9e3779b97f4a7c15 (mod 2^64): the sum s of the hash's four 16-bit fields
 * minus 131070 (an Irwin-Hall(4) draw with mean 0) times
 * c = (float)(std * sqrt(3) / 65536), one f32 multiply. Matrices are then quantized
 * to Q8_0 by the rule of kanso_quantize_q8_0; norms = 1. Every value is an exact
 * integer times one rounding, so a host restatement reproduces the weights bit
 * for bit. */
int kanso_model_init_random(kanso_model* model, uint64_t seed, float std);

/* Reads one weight back to host memory in kanso_model_set_weight's format (GGUF
 * Q8_0 bytes of a matrix, f32 norm vectors). No reference counterpart: the
 * reference keeps its weights in host tensors (src/weights.rs:33-45). */
int kanso_model_get_weight(kanso_model* model, uint32_t kind, uint32_t layer, void* host_out,
                           size_t bytes);

/* Allocates the F32 KV pool: num_blocks blocks of block_size tokens per layer, and
 * step buffers for up to max_tokens rows and max_seqs sequences per forward. */
int kanso_model_alloc_kv(kanso_model* model, uint32_t num_blocks, uint32_t block_size,
                         uint32_t max_tokens, uint32_t max_seqs);

/* kanso_model_alloc_kv with a pool kind (Engine::new_with_budget_and_kv's kv_mode,
 * src/engine.rs:62-100): KANSO_KV_F32, or a 1-byte pool (INT8 / FP8 with one f32
 * scale per token-head row, Q8_0 with one f16 scale per 32 elements). With a
 * 1-byte pool each layer's new K / V rows go through the fused append + quantize
 * (kanso_kv_append) and the attention reads the pool in that kind;
 * kanso_model_kv_pool / kanso_model_read_kv_rows then report an error. */
int kanso_model_alloc_kv_quant(kanso_model* model, uint32_t num_blocks, uint32_t block_size,
                               uint32_t max_tokens, uint32_t max_seqs, uint32_t kv_dtype);

/* Device pointers of layer `layer`'s K and V pools ([num_blocks][bs][kv_heads][64]). */
int kanso_model_kv_pool(kanso_model* model, uint32_t layer, float** k_pool, float** v_pool);

/* Copies the K and V rows of pool slots slots[0..n) of layer `layer` to host
 * arrays k_out / v_out ([n][kv_heads][64] f32) (KvStorageKind::read_kv_token,
 * src/kv_cache/kind.rs:400-411). Synchronous. */
int kanso_model_read_kv_rows(kanso_model* model, uint32_t layer, const uint64_t* slots,
                             uint32_t n, float* k_out, float* v_out);

/* Erases blocks (host array) in every layer's K and V pool (allocate_zeroed,
 * src/kv_cache/mod.rs:25-35). */
int kanso_model_reset_blocks(kanso_model* model, const uint32_t* blocks, uint32_t num_blocks,
                             kanso_stream_t stream);

/* One batched forward (Model::forward_batch, src/model.rs:1360-1380) of a step
 * given as a compact plan (host arrays, as for kanso_pack_step: token_offset + pos
 * is taken modulo 2^32, so an arena holding only this step's tokens uses
 * token_offset = arena_index - start_pos). Packs on the device, runs every layer,
 * and writes next_tokens[s] (host) = greedy token of sequence s's last row;
 * logits [S][vocab] (device) too when non-NULL. Synchronises `stream`. */
int kanso_model_forward(kanso_model* model, const kanso_seq_plan* plan, uint32_t num_seqs,
                        const uint32_t* token_arena, uint32_t token_arena_len,
                        const uint32_t* table_arena, uint32_t table_arena_len, float* logits,
                        uint32_t* next_tokens, kanso_stream_t stream);

/* Model::forward_batch_all_rows (src/model.rs:1382-1410, RowSelection::EveryToken):
 * the same forward, but the final norm, lm_head and greedy argmax run on every new
 * token, the rows a speculative verifier scores its candidates with. next_tokens
 * (host) has T = sum of q_len entries, in plan order; logits [T][vocab] (device)
 * when non-NULL. Synchronises `stream`. */
int kanso_model_forward_all_rows(kanso_model* model, const kanso_seq_plan* plan, uint32_t num_seqs,
                                 const uint32_t* token_arena, uint32_t token_arena_len,
                                 const uint32_t* table_arena, uint32_t table_arena_len, float* logits,
                                 uint32_t* next_tokens, kanso_stream_t stream);

/* Engine::new_with_budget (src/engine.rs:46-125): a block pool of total_blocks,
 * a prefix cache, max_running sequences, token_budget tokens per step. model may be
 * NULL: the engine then plans and commits with a deterministic stand-in token
 * (kanso_engine_dry_token) instead of a forward — the scheduler alone, for tests. */
int kanso_engine_create(kanso_model* model, uint32_t max_running, uint32_t total_blocks,
                        uint32_t block_size, uint32_t token_budget, uint32_t dry_vocab,
                        kanso_engine** out);
int kanso_engine_destroy(kanso_engine* engine);

/* add_request_with_stops (src/engine.rs:138-170): returns the request id. */
int kanso_engine_add_request(kanso_engine* engine, const uint32_t* prompt, uint32_t prompt_len,
                             uint32_t max_tokens, const uint32_t* stop_ids, uint32_t num_stop,
                             uint64_t* request_id);

/* One StepOutput (src/engine.rs:11-16). */
typedef struct {
    uint64_t request_id;
    uint32_t token_id;
    uint32_t is_finished;
} kanso_step_output;

/* Engine::step (src/engine.rs:213-505): plan, one forward, commit, retire. Writes
 * up to capacity outputs (in emit order) and their count. */
int kanso_engine_step(kanso_engine* engine, kanso_step_output* outputs, uint32_t capacity,
                      uint32_t* num_outputs);

/* The flattened batch of the last step (engine.rs:376-402, before padding):
 * counts into sizes[0..3] = {tokens, sequences, table entries, sample rows}; when
 * the arrays are non-NULL they receive tokens/positions/slots [T], context_lens /
 * query_lens [S], table_lens [S] and the concatenated tables, sample rows. */
int kanso_engine_last_plan(kanso_engine* engine, uint32_t* sizes, uint32_t* tokens,
                           uint32_t* positions, uint64_t* slots, uint32_t* context_lens,
                           uint32_t* query_lens, uint32_t* table_lens, uint32_t* tables,
                           uint32_t* sample_rows);

/* Counters: {waiting, running, free blocks, unfinished, sequences, prefix hits,
 * prefix lookups, prefix matched tokens, prompt tokens admitted, steps}. */
int kanso_engine_stats(kanso_engine* engine, uint64_t* stats10);

/* cancel_request (src/engine.rs:516-531); *found = 0 when no such request is live. */
int kanso_engine_cancel(kanso_engine* engine, uint64_t request_id, uint32_t* found);
/* drain_finished (src/engine.rs:511-515). */
int kanso_engine_drain_finished(kanso_engine* engine, uint32_t* dropped);

/* The stand-in token of the model-less engine for (request id, position). */
uint32_t kanso_engine_dry_token(uint64_t request_id, uint32_t position, uint32_t vocab);

/* Timing of the library's own kernels with HIP events on the launch stream.
 * When enabled, every launch of the named kernel is bracketed by events and the
 * elapsed times are summed. Names: "attention" (stage 1), "reduce", "gemv",
 * "append", "pack". */
int kanso_set_profiling(kanso_ctx* ctx, int enabled);
int kanso_get_kernel_time(kanso_ctx* ctx, const char* name, double* total_ms,
                          uint64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* KANSO_HIP_H */
