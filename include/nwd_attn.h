/*
 * nwd_attn.h — C ABI of the MI355X (gfx950) decode-attention path.
 *
 * This library replaces the two leaf kernels that the reference engine
 * dispatches for every attention layer of every token:
 *
 *   kernels/kv_append.wgsl    main  :12-18  (dispatched twice, K then V,
 *                                            engine/runtime.js:389-390)
 *   kernels/sparse_attn.wgsl  main  :31-114 (dispatched with H workgroups,
 *                                            engine/runtime.js:391)
 *
 * and keeps their buffer contract: a query buffer, a K cache, a V cache, a
 * position, and an output buffer (bind groups built at engine/runtime.js:331-333).
 * The reference passes the position through two uniforms,
 * uKv.seq = seq and uAttn.seq = seq + 1 (engine/runtime.js:451-452). Here the
 * position lives in a device int32 buffer, one entry per sequence:
 *
 *   pos[b]  = index at which the newest token of sequence b is (or was) written;
 *   L_b     = pos[b] + 1 keys are attended (keys 0..pos[b], all visible, which
 *             is the reference's causal rule, kernels/sparse_attn.wgsl:9).
 *
 * Differences from the reference, all requested by the caller's descriptor:
 *   - the cache is fp16 and head-major per sequence (see nwd_cache_offset);
 *   - Q and O may be fp16 or fp32 (the reference is fp32 only,
 *     kernels/sparse_attn.wgsl:19-22); arithmetic is fp32 either way;
 *   - there is a batch dimension and no 256-key cap
 *     (kernels/sparse_attn.wgsl:29, engine/config.js:24);
 *   - a causal chunked-prefill entry point replaces the reference's
 *     token-by-token prefill (engine/runtime.js:640-643) with one call.
 *
 * All buffers are caller-owned device memory. Every call only enqueues work
 * on the given HIP stream (0 = the null stream); nothing synchronises unless
 * documented. A context is not thread-safe and its calls must be ordered on
 * one stream: the split-K workspace belongs to the context.
 */
#ifndef NWD_ATTN_H
#define NWD_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. 0 is success; every failing call also sets nwd_last_error. */
enum {
  NWD_OK = 0,
  NWD_ERR_INVALID = 1,     /* bad descriptor, null pointer, bad shape      */
  NWD_ERR_UNSUPPORTED = 2, /* shape the kernels are not built for           */
  NWD_ERR_CAPACITY = 3,    /* a position would write/read past max_seq,
                              or batch > max_batch (engine/runtime.js:448)  */
  NWD_ERR_HIP = 4,         /* a HIP runtime call failed                     */
  NWD_ERR_DEVICE = 5       /* a kernel flagged an out-of-range device
                              position (reported by nwd_device_status)      */
};

/* Element types of Q, O and of the new K/V rows. The cache is always fp16. */
enum { NWD_F32 = 0, NWD_F16 = 1 };

/* Descriptor. Mirrors the attention Params uniform {n_heads, n_kv_heads,
 * head_dim, seq} (kernels/sparse_attn.wgsl:12-17, engine/runtime.js:182) plus
 * the allocation sizes the engine derives from engine/config.js:10-12,24. */
typedef struct nwd_desc {
  int32_t n_heads;     /* H, query heads (32 in the benchmark shapes, 40 in
                          the Nano-4B model, engine/config.js:10)           */
  int32_t n_kv_heads;  /* Hkv; H must be a multiple of Hkv, any group
                          G = H/Hkv (sparse_attn.wgsl:38-39)                */
  int32_t head_dim;    /* D, 1 .. 512 (128 in engine/config.js:12). D = 128
                          with G from 1 to 8 runs the kernels built for
                          those shapes; decodes at D = 64 (G 1 to 8, also
                          on the matrix-core kernel) and D = 256 (G 1 to
                          5) run the dot-product
                          split kernel built for those sizes, and at the
                          other multiples of 8 up to 256 its form for rows
                          padded to 64, 128 or 256 dims, there with G = 3,
                          6, 7 as G = 4, 8, 8 on zero-padded query rows
                          (buffers allocated by nwd_create); larger groups
                          run as several built groups per KV head or on
                          query rows padded to such groups (a K/V slab above
                          1 GiB, max_seq * D * 2 bytes, takes the general
                          kernels);
                          prefills at D = 64 and 256, and at the other
                          multiples of 8 up to 256, run MFMA prefill
                          kernels built for D = 64, 128 and 256 on rows
                          padded to those dims (other groups as for
                          decode);
                          every other (D, G) runs the general kernels, with
                          the same contract and cache layout (a coverage
                          path, not tuned like the others)                   */
  int32_t max_seq;     /* cache capacity in tokens per sequence, at most
                          4194304 (2^22)                                    */
  int32_t max_batch;   /* sequences per call                                */
  int32_t q_dtype;     /* NWD_F16 or NWD_F32                                */
  int32_t o_dtype;     /* NWD_F16 or NWD_F32                                */
  int32_t kv_dtype;    /* type of the new K/V rows given to nwd_kv_append   */
  float scale;         /* softmax scale; 0 means 1/sqrt(D) as the reference
                          computes it (kernels/sparse_attn.wgsl:42)         */
} nwd_desc;

typedef struct nwd_ctx nwd_ctx;

/* Creates a context on the current HIP device and allocates its split-K
 * workspace and status word once (the reference allocates once too,
 * engine/runtime.js:109-211). Replaces the attention slice of
 * DecodeEngine._compile/_alloc (engine/runtime.js:101-102,170-173,182-183). */
int nwd_create(const nwd_desc* desc, nwd_ctx** out_ctx);

/* Frees the context's own device memory (never the caller's buffers). */
void nwd_destroy(nwd_ctx* ctx);

/* Message for the last failing call on ctx (or for nwd_create when ctx is
 * NULL). Never NULL. */
const char* nwd_last_error(const nwd_ctx* ctx);

/* SHA-256 (hex) of the sources this library was built from: every file under
 * csrc/ (its .hip and .h files, not those of csrc/bench/, in name order,
 * each as its relative path, a NUL, its bytes) and include/nwd_attn.h. A provenance check with no
 * counterpart in the reference: a host compares it with the sources on disk
 * to know that the library it loaded is the one those sources build. */
const char* nwd_source_hash(void);

/* Bytes of ONE cache (K or V) for max_batch sequences of max_seq tokens:
 * max_batch * n_kv_heads * max_seq * head_dim * 2. The reference's cache is
 * f32 [maxSeq][kvHeads][headDim] (engine/runtime.js:171-172). */
size_t nwd_cache_bytes(const nwd_ctx* ctx);

/* Element index of (sequence b, token t, kv head h, dim d) in a cache:
 * ((b * n_kv_heads + h) * max_seq + t) * head_dim + d. Each (b, h) owns one
 * contiguous [max_seq][head_dim] fp16 slab, so a run of keys is one
 * contiguous stream. The reference indexes (t * n_kv + h) * hd + d
 * (kernels/sparse_attn.wgsl:49,107, kernels/kv_append.wgsl:17). */
int64_t nwd_cache_offset(const nwd_ctx* ctx, int32_t b, int32_t t, int32_t h,
                         int32_t d);

/* Fused K+V append; replaces kv_append.wgsl main (:12-18) dispatched once for
 * K and once for V (engine/runtime.js:389-390). For each sequence b < batch
 * and new token j < n_tokens, copies row k_new[b][j][:][:] and
 * v_new[b][j][:][:] ([n_kv_heads][head_dim], type desc.kv_dtype) into the
 * caches at token pos[b] + j. fp16 rows are copied bit for bit; fp32 rows are
 * rounded to nearest-even fp16. pos is a device int32[batch]. A position with
 * pos[b] + n_tokens > max_seq is not written; the kernel records it in the
 * status word (nwd_device_status). One launch. */
int nwd_kv_append(nwd_ctx* ctx, const void* k_new, const void* v_new,
                  void* k_cache, void* v_cache, const int32_t* pos,
                  int32_t batch, int32_t n_tokens, void* stream);

/* Decode attention; replaces sparse_attn.wgsl main (:31-114). For sequence b
 * and query head h: out[b][h][:] = softmax(q[b][h] . K[b][h/G][0..L_b)^T *
 * scale) . V[b][h/G][0..L_b), L_b = pos[b] + 1. q and out are
 * [batch][n_heads][head_dim] in desc.q_dtype / desc.o_dtype. max_len bounds
 * max_b L_b from the host side (the reference host knows seq, runtime.js:452);
 * it only sizes the split-K grid: results are exact for any device positions,
 * and 0 means max_seq. Long contexts are split across CUs into partial
 * (max, sum, o) records that are then merged (the argmax_partial /
 * argmax_merge pattern, kernels/argmax_partial.wgsl:16-52,
 * kernels/argmax_merge.wgsl:8-42); see nwd_set_decode_merge. */
int nwd_decode_attn(nwd_ctx* ctx, const void* q, const void* k_cache,
                    const void* v_cache, const int32_t* pos, void* out,
                    int32_t batch, int32_t max_len, void* stream);

/* One attention-layer step: the fused form of kv_append for K and V followed
 * by sparse_attn, which the reference encodes as three dispatches in one
 * compute pass (engine/runtime.js:389-391); here one launch, plus the merge
 * kernel when the context is split (see nwd_set_decode_merge). Appends one new
 * token per sequence (k_new / v_new [batch][n_kv_heads][head_dim], type
 * desc.kv_dtype, written at pos[b] exactly as nwd_kv_append does) and
 * attends over L_b = pos[b] + 1 keys including it; q and out as in
 * nwd_decode_attn. A position outside [0, max_seq) writes nothing and is
 * reported by nwd_device_status. */
int nwd_append_decode(nwd_ctx* ctx, const void* q, const void* k_new,
                      const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* pos, void* out, int32_t batch,
                      int32_t max_len, void* stream);

/* Allocation-free form of nwd_append_decode, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. It has no counterpart in the reference.
 * It takes the descriptor instead of a context and needs no nwd_create: the
 * split-K records live in a static 16 MiB device array of the library (one
 * per GPU, held until the process ends), so a call whose records would not
 * fit (batch * n_heads * splits > 32262 when it splits) fails with
 * NWD_ERR_CAPACITY before any launch; records hold 128 floats up to head_dim
 * 128, 256 up to 256 (multiples of 8), head_dim otherwise. The merge always
 * runs as a separate kernel. Results are bit-identical to nwd_append_decode
 * on a context made from the same descriptor (default merge form, automatic
 * split count), except for the groups a context runs on padded query rows
 * (3, 6 and 7 at head sizes other than 64 and 128, and larger groups with no
 * built divisor), which take the general kernels here (no padded buffers):
 * the same results within fp32 rounding.
 * status, if not NULL, is a caller-owned device int32 that gets bit 1 OR-ed
 * in when a position is outside [0, max_seq) (nothing is written there and
 * attention is clamped, as in nwd_append_decode); with NULL such a position
 * is not reported. All calls on one GPU share its scratch: calls that may
 * run at the same time on one GPU (on different streams) race. */
int nwd_append_decode_noalloc(const nwd_desc* desc, const void* q, const void* k_new,
                              const void* v_new, void* k_cache, void* v_cache,
                              const int32_t* pos, void* out, int32_t batch,
                              int32_t max_len, int32_t* status, void* stream);

/* Causal chunked prefill; replaces the token-by-token prefill of
 * engine/runtime.js:640-643 (each prompt token runs kv_append then
 * sparse_attn). The n_new new rows must already be in the caches at tokens
 * pos0[b] .. pos0[b] + n_new - 1 (nwd_kv_append with n_tokens = n_new).
 * Query i of sequence b attends keys 0 .. pos0[b] + i. q and out are
 * [batch][n_new][n_heads][head_dim]. QK^T and PV run on fp16 MFMA with fp32
 * accumulation: an fp16 q enters exact and its scores are scaled in fp32;
 * an fp32 q is scaled by scale * log2(e) and carried as fp16 high and low
 * parts (~22 bits). A scaled fp32 q element beyond the fp16 range (65504)
 * makes nwd_device_status report NWD_ERR_DEVICE (head sizes up to 256 run
 * these kernels, or head-64 and head-256 forms of them, on rows padded with
 * zeros to 64, 128 or 256 dims, and padded groups on padded query rows, in
 * sub-chunks).
 * The shapes of the general kernels
 * (see nwd_desc.head_dim) compute in fp32 on the vector units instead. A chunk
 * outside the cache (pos0[b] < 0 or pos0[b] + n_new > max_seq) is flagged in
 * the device status and run at the nearest valid pos0. max_len bounds
 * pos0[b] + n_new (0 means max_seq). */
int nwd_prefill_attn(nwd_ctx* ctx, const void* q, const void* k_cache,
                     const void* v_cache, const int32_t* pos0, void* out,
                     int32_t batch, int32_t n_new, int32_t max_len,
                     void* stream);

/* Synchronises the stream, returns NWD_OK if no kernel since the last call
 * flagged an out-of-range device position (else NWD_ERR_DEVICE), and clears
 * the flag. A library built with -DNWD_CHECK also flags, and drops, any
 * kernel store whose address falls outside its buffer. The reference throws at the host guard instead
 * (engine/runtime.js:448). */
int nwd_device_status(nwd_ctx* ctx, void* stream);

/* Number of split-K partitions nwd_decode_attn launches for (batch, max_len),
 * exposed so tests can force both the single-pass and the merged path. */
int32_t nwd_decode_splits(const nwd_ctx* ctx, int32_t batch, int32_t max_len);

/* Overrides the split count chosen by nwd_decode_attn (0 restores the
 * automatic choice); on shapes whose prefill runs the general kernels (see
 * nwd_desc.head_dim) it also sets nwd_prefill_attn's. Values are clamped to [1, 256]. Results do not
 * depend on it beyond fp32 reordering. */
int nwd_set_decode_splits(nwd_ctx* ctx, int32_t n_splits);

/* Chooses where split-K records are merged: 1 in a separate merge kernel
 * launched after the split kernel (the two-dispatch shape of argmax_partial /
 * argmax_merge, engine/runtime.js:398-399); 0 inside the split kernel, by the
 * last workgroup of each (sequence, kv head) to finish (of each (sequence,
 * query head) when the call runs one workgroup per query head); negative restores the
 * default, the separate kernel (measured faster on MI355X at 4K and 32K
 * keys). Same results, bit for bit. The general kernels always use the
 * separate merge; this and the two knobs below do not apply to them (at
 * D = 64 all three apply; at 256 and on the padded head forms this and the
 * layout knob apply, the kernel knob does not: only the dot-product kernel
 * is built for those sizes). */
int nwd_set_decode_merge(nwd_ctx* ctx, int32_t separate_kernel);

/* Chooses the split kernel of later decode calls at head sizes 128 and 64
 * (the workgroup form of sparse_attn.wgsl main,
 * kernels/sparse_attn.wgsl:31-114): 0 the dot-product
 * kernel (VALU, whose work per key grows with the group size G), 1 the
 * matrix-core kernel (MFMA, the same work for every G), -1 restores the
 * default, which takes the matrix-core kernel for calls that run one
 * workgroup per KV head with G >= 5, or with G = 4 and either batch >= 2 or
 * splits of at least 512 keys whose workgroups all run at once (where it
 * measured faster on MI355X), the dot-product kernel otherwise. Same records
 * and merges; results agree within fp32 rounding (both accumulate in fp32),
 * not bit for bit. */
int nwd_set_decode_kernel(nwd_ctx* ctx, int32_t kernel);

/* Chooses how later decode calls lay the keys over the split workgroups
 * (a tuning knob with no counterpart in the reference, whose one workgroup
 * per query head reads every key, kernels/sparse_attn.wgsl:45-58): 0
 * contiguous, each split owns one range of keys; 1 strided, split s owns
 * the 64-key blocks (32 for the dot-product kernel) s, s + n_splits, ..., so
 * the splits of a KV head read neighbouring blocks at any moment; -1
 * restores the default: strided for batches of two or more sequences,
 * contiguous for one (measured on MI355X). Results agree within fp32
 * rounding (the keys a split sums differ), not bit for bit. */
int nwd_set_decode_layout(nwd_ctx* ctx, int32_t layout);

/* Measurement hook (no counterpart in the reference, whose split/merge
 * kernels are timed only as a whole step, bench/engine.js:70-137): while set,
 * the split kernel of every decode call on ctx is launched so that the HIP
 * runtime records start_event when it begins and stop_event when it ends
 * (hipEvent_t handles created by the caller with timing enabled), which
 * separates its duration from the merge kernel's. NULL, NULL turns it off.
 * Not for calls under HIP graph capture. */
int nwd_set_kernel_events(nwd_ctx* ctx, void* start_event, void* stop_event);

/* ---------------------------------------------------------------------
 * 4-bit projections around the path: the producer of q / k / v and the
 * consumer of the attention output.
 * ------------------------------------------------------------------- */

/* One 4-bit projection [K -> n] in the reference's MatMulNBits format
 * (engine/weights.js:99-104, engine/weight-index.json; read by
 * kernels/matmul_nbits_sg.wgsl:15-18). Weight (c, k) of block blk = k / 32
 * is (nib - zp) * scale with nib the low nibble of byte (k % 32) / 2 of
 * quant[c][blk] for even k (high nibble for odd), scale = scales[c][blk] and
 * zp nibble c * n_blocks + blk of the packed zero points (low nibble first,
 * matmul_nbits_sg.wgsl:24-27). */
typedef struct nwd_q4_weight {
  const void* quant;     /* uint8 [n][n_blocks][16], 16-byte aligned         */
  const float* scales;   /* float [n][n_blocks]                              */
  const void* zp;        /* uint8 [(n * n_blocks + 1) / 2]                   */
  int32_t n;             /* output columns N                                 */
  int32_t n_blocks;      /* K / 32, 1..256                                   */
} nwd_q4_weight;

enum {
  NWD_Q4_PLAIN = 0,      /* y = W . a                                        */
  NWD_Q4_RELU2 = 1,      /* y = max(W . a, 0)^2 (matmul_nbits_sg.wgsl epilogue
                            1, :76-79,125-127)                               */
  NWD_Q4_ACCUMULATE = 2  /* y = y + W . a: a projection followed by the
                            residual add of kernels/add.wgsl:15-18, as o_proj
                            and L-add run at engine/runtime.js:392-393     */
};

/* matmul_nbits_sg.wgsl main (:81-137) for `batch` activation rows:
 * y[b][n] = epilogue(W . a[b]). a is [batch][32 * n_blocks] f32 (16-byte
 * aligned), y [batch][n] f32. Dispatched as ceil(N / 4) workgroups by the
 * reference (engine/runtime.js:359-361); here the library picks the grid. */
int nwd_q4_gemv(nwd_ctx* ctx, const float* a, const nwd_q4_weight* w, float* y,
                int32_t batch, int32_t epilogue, void* stream);

/* The attention layer's q / k / v projections and kv_append in one launch:
 * the dispatches L-q, L-k, L-v, L-kvK and L-kvV of engine/runtime.js:386-390
 * (matmul_nbits_sg.wgsl three times, then kv_append.wgsl:12-18 for k and
 * v). x is [batch][K] f32 (the normalised hidden state, 16-byte aligned); wq
 * has n_heads * head_dim columns, wk and wv n_kv_heads * head_dim, all with
 * the same K. q_out gets [batch][n_heads][head_dim] in desc.q_dtype (the q
 * input of nwd_decode_attn); the new k and v rows are rounded to fp16 (to
 * nearest even, as nwd_kv_append does) into the caches at pos[b]. A position
 * outside [0, max_seq) writes no cache row and sets the device status
 * (nwd_device_status). batch <= max_batch. head_dim must be a multiple of 4
 * and n_heads * head_dim, n_kv_heads * head_dim multiples of 16 (a
 * workgroup's 16 columns lie in one of q, k, v); else NWD_ERR_UNSUPPORTED. */
int nwd_qkv_append(nwd_ctx* ctx, const float* x, const nwd_q4_weight* wq,
                   const nwd_q4_weight* wk, const nwd_q4_weight* wv, void* q_out,
                   void* k_cache, void* v_cache, const int32_t* pos, int32_t batch,
                   void* stream);

/* The greedy token pick: kernels/argmax_partial.wgsl (:16-52) over 256
 * slices of ceil(n / 256) logits, then kernels/argmax_merge.wgsl (:8-42),
 * as dispatched at engine/runtime.js:398-399. out[b] gets the index the
 * reference returns for row b of x [batch][n] f32, including its tie order
 * (the smaller step within a thread, then the smaller bit-reversed thread
 * and slice positions of its two reduction trees), NaN never winning, and
 * 0 when no value exceeds -3.402823466e38. Uses the context's workspace. */
int nwd_argmax(nwd_ctx* ctx, const float* x, int32_t n, uint32_t* out, int32_t batch,
               void* stream);

/* lm_head and the greedy pick: the dispatches lm-head, argmax0 and argmax1
 * of engine/runtime.js:397-399 (matmul_nbits_sg.wgsl then the two argmax
 * kernels), with the partial argmax in the GEMV's epilogue. h is
 * [batch][K] f32 (16-byte aligned, the final-norm output), w the 4-bit
 * lm_head [K -> vocab]; out[b] gets the token index, with nwd_argmax's
 * semantics over the logits; logits, if not NULL, gets them [batch][vocab]
 * f32. */
int nwd_lm_head_argmax(nwd_ctx* ctx, const float* h, const nwd_q4_weight* w, float* logits,
                       uint32_t* out, int32_t batch, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NWD_ATTN_H */
