// nwd_internal.h — launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nwd {

// Shapes fixed at context creation.
struct Shape {
  int n_heads;     // H
  int n_kv;        // Hkv
  int group;       // H / Hkv
  int cap;         // max_seq
  int q16;         // Q is fp16 (else fp32)
  int o16;         // O is fp16 (else fp32)
  int kv16;        // new K/V rows are fp16 (else fp32)
  float qk_scale;  // softmax scale (1/sqrt(D) by default)
  int head_dim;    // D
};

// Head sizes the general-shape kernels take (sparse_attn.wgsl:12-17 takes
// any; a row of q and the partial output stay in LDS).
constexpr int kMaxHeadDim = 512;
// Floats per split-K record at head size D: the split kernels and the MFMA
// prefills keep the dims of the kernel they run on (128 for the multiples of
// 8 up to 128, 256 above), the general kernels D.
inline int record_width(int head_dim) {
  if (head_dim % 8 == 0 && head_dim <= 256) return head_dim <= 128 ? 128 : 256;
  return head_dim;
}

// Split-K workspace owned by the context.
struct Workspace {
  float* part_o;     // [records][D] unnormalised partial outputs
  float2* part_ml;   // [records] (running max in log2 units, sum of weights)
  int64_t records;   // capacity in records
  int* counters;     // merge arrival tickets per (sequence, query head group), zero between calls
  int* status;       // device status word (kStatus* bits)
};

// One decode call. k_new/v_new non-null = fused append of one token per
// sequence at pos[b] before attending.
struct DecodeCall {
  const void* q;
  void* k_cache;
  void* v_cache;
  const int32_t* pos;
  void* out;
  const void* k_new;
  const void* v_new;
  int batch;
  int nsplit;
  int span;  // host bound on the keys attended (max_len), partitions the splits
  int fused_merge;  // merge in the split kernel (else a separate merge kernel)
  int kernel;       // -1 the launch's choice, 0 dot-product (VALU), 1 matrix-core
  int layout;       // keys over the splits: 0 contiguous ranges, 1 interleaved blocks
  void* ev_start;   // optional hipEvent_t pair recorded around the split kernel
  void* ev_stop;
};

hipError_t launch_kv_append(const Shape& s, const void* k_new, const void* v_new,
                            void* k_cache, void* v_cache, const int32_t* pos,
                            int batch, int n_tokens, int* status,
                            hipStream_t stream);

// The group the decode and prefill kernels run a group of `group` query
// heads as, with *kv_rep such groups per KV head: the group itself for 1, 2,
// 4, 5 and 8 (8 only up to head size 128), at head sizes 128 and 64 for
// every group up to 8, and for 3 at 256; for larger groups a built size that divides them into
// ceil(group / largest built size) groups; 0 when the group must be padded
// first (padded_group).
int kernel_group(int head_dim, int group, int* kv_rep);

// Shapes launch_decode takes: a head size that is a multiple of 8 up to 256
// and a group kernel_group maps. 64, 128 and 256 run kernels built for
// them, the other sizes those kernels' padded form.
bool split_decode_shape(int head_dim, int group);

// nsplit == 1 writes `out` directly; otherwise partial records then a merge.
hipError_t launch_decode(const Shape& s, const DecodeCall& c, const Workspace& ws,
                         hipStream_t stream);

// Largest batch x query heads for which a single-split decode runs one
// workgroup per query head (one per CU); the split rule uses it too. Beyond
// it the G-fold K/V reads cost more than the shorter chains save: 153 keys,
// 32 query heads, per append + attend step, B = 16: 8.4 against 6.7 us,
// B = 32: 13.4 against 7.2 (B = 1-8 gain or tie).
constexpr int kSubSplitMaxWorkgroups = 256;

// Head sizes launch_prefill takes: the multiples of 8 up to 256. 128 and 256
// run kernels built for them, the others those kernels' rows padded with
// zeros (below 128: nwd_prefill.hip; above: nwd_prefill_wide.hip).
bool prefill_head_dim(int head_dim);
bool prefill_wide_head_dim(int head_dim);  // 136 .. 256
hipError_t launch_prefill_wide(const Shape& s, const void* q, const void* k_cache,
                               const void* v_cache, const int32_t* pos0, void* out, int batch,
                               int n_new, int max_len, const Workspace& ws, hipStream_t stream);

hipError_t launch_prefill(const Shape& s, const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* pos0, void* out,
                          int batch, int n_new, int max_len, const Workspace& ws,
                          hipStream_t stream);

// Largest decode split count supported for `batch` sequences by `ws`.
int max_decode_splits(const Shape& s, const Workspace& ws, int batch);

// Groups kernel_group does not map run as a padded group (padded_group; 0
// for groups that need no padding): 3 as 4, 6 and 7 as 8 (at head sizes
// other than 128 and 64), larger groups as the next multiple of 8 (of 5 above head
// size 128), where launch_decode takes the padded group at the head size
// (padded_decode_shape), their
// query rows copied into a padded layout (q_pad, [batch][Hkv][padded
// group][D], the call's q dtype) and the real rows copied out of out_pad
// afterwards.
int padded_group(int head_dim, int group);
bool padded_decode_shape(int head_dim, int group);
Shape padded_shape(const Shape& s);
hipError_t launch_padded_decode(const Shape& s, const DecodeCall& c, const Workspace& ws,
                                void* q_pad, void* out_pad, hipStream_t stream);

// The prefill of those groups on the prefill kernels of groups 4 / 8 (head
// sizes prefill_head_dim takes): the chunk goes through in sub-chunks of
// chunk_tokens tokens, each padded into q_pad
// ([batch][chunk_tokens][Hkv][padded group][D]), its first positions in
// pos_sub ([batch]), its output unpadded from out_pad.
struct PadBuffers {
  void* q_pad;
  void* out_pad;
  int32_t* pos_sub;
  int chunk_tokens;
};
hipError_t launch_padded_prefill(const Shape& s, const void* q, const void* k_cache,
                                 const void* v_cache, const int32_t* pos0, void* out, int batch,
                                 int n_new, int max_len, const Workspace& ws, const PadBuffers& pb,
                                 hipStream_t stream);

// Query heads one general-shape workgroup serves (the same K/V rows read once
// for all of them): up to 8 at D <= 128, 4 at D <= 256, 2 beyond, 1 when D
// is not a multiple of 8; never more than the group.
int general_heads_per_workgroup(int head_dim, int group);

// Decode (prefill = 0, n_new = 1, pos = the newest token's index) or causal
// prefill (prefill = 1, pos = pos0) of the general-shape kernels over rows
// [batch][n_new][H]: one workgroup per split and chunk of a group's heads,
// split-K records of D floats per row in ws, then a merge launch when
// nsplit > 1. span bounds the keys from the host side and partitions the
// splits.
hipError_t launch_general_attn(const Shape& s, const void* q, const void* k_cache,
                               const void* v_cache, const int32_t* pos, void* out, int batch,
                               int n_new, int prefill, int span, int nsplit, const Workspace& ws,
                               void* ev_start, void* ev_stop, hipStream_t stream);

// One 4-bit projection [K -> n] in the reference's format (K = 32 * n_blocks).
struct Q4Mat {
  const uint8_t* quant;   // [n][n_blocks][16]
  const float* scales;    // [n][n_blocks]
  const uint8_t* zp;      // 4-bit zero points, flat index col * n_blocks + blk
  int n;
};

// Largest K = 32 * n_blocks the 4-bit kernels accept (activation blocks are
// held in registers, four per lane).
constexpr int kQ4MaxBlocks = 256;

enum Q4Epilogue { kQ4None = 0, kQ4Relu2 = 1, kQ4Accumulate = 2 };

// y[b][n] = epilogue(dequant(W) . x[b]) for b < batch; x [batch][K] f32.
hipError_t launch_q4_gemv(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                          int epilogue, hipStream_t stream);

// The attention layer's q/k/v projections of x [batch][K] with the new K/V
// rows rounded to fp16 straight into the caches at pos[b] (q to q_out,
// [batch][H][D] in the context's q dtype).
hipError_t launch_qkv_append(const Shape& s, const float* x, const Q4Mat& wq, const Q4Mat& wk,
                             const Q4Mat& wv, int n_blocks, void* q_out, void* k_cache,
                             void* v_cache, const int32_t* pos, int batch, int* status,
                             hipStream_t stream);

// The greedy pick of kernels/argmax_partial.wgsl + argmax_merge.wgsl over
// x [batch][n]: one 64-bit record per chunk of logits in `records`, then a
// merge per row into out[b]. records needs argmax_records_per_row(n) * batch
// entries.
int argmax_records_per_row(int n);
hipError_t launch_argmax(const float* x, int n, uint32_t* out, int batch,
                         unsigned long long* records, hipStream_t stream);
hipError_t launch_argmax_merge(const unsigned long long* records, int per_row, int n,
                               uint32_t* out, int batch, hipStream_t stream);

// lm_head (a 4-bit projection of x [batch][K] to w.n logits) with the
// argmax partial in its epilogue: one record per 16 logits, then the merge.
// logits (optional) gets the projection. records needs
// q4_argmax_records_per_row(w.n) * batch entries.
int q4_argmax_records_per_row(int n);
hipError_t launch_q4_argmax(const float* x, const Q4Mat& w, int n_blocks, float* logits,
                            uint32_t* out, int batch, unsigned long long* records,
                            hipStream_t stream);

}  // namespace nwd
