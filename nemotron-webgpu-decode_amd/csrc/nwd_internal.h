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
};

// Split-K workspace owned by the context.
struct Workspace {
  float* part_o;     // [records][D] unnormalised partial outputs
  float2* part_ml;   // [records] (running max in log2 units, sum of weights)
  int64_t records;   // capacity in records
  int* counters;     // [max_batch][n_kv] merge arrival tickets (zero between calls)
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
};

hipError_t launch_kv_append(const Shape& s, const void* k_new, const void* v_new,
                            void* k_cache, void* v_cache, const int32_t* pos,
                            int batch, int n_tokens, int* status,
                            hipStream_t stream);

// nsplit == 1 writes `out` directly; otherwise partial records then a merge.
hipError_t launch_decode(const Shape& s, const DecodeCall& c, const Workspace& ws,
                         hipStream_t stream);

hipError_t launch_prefill(const Shape& s, const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* pos0, void* out,
                          int batch, int n_new, int max_len, const Workspace& ws,
                          hipStream_t stream);

// Largest decode split count supported for `batch` sequences by `ws`.
int max_decode_splits(const Shape& s, const Workspace& ws, int batch);

}  // namespace nwd
