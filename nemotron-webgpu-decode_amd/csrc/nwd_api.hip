// nwd_api.hip — the C ABI of libnwd_attn (declared in include/nwd_attn.h).
//
// Host-side validation and launch planning. Kernels never see a shape the
// checks below have not accepted, and the context owns the only device
// memory the library allocates (split-K workspace and the status word), once,
// at nwd_create — as the reference engine allocates its buffers once in
// DecodeEngine._alloc (engine/runtime.js:109-211).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/nwd_attn.h"
#include "nwd_common.h"
#include "nwd_internal.h"

// Device scratch of nwd_append_decode_noalloc: a status word, then the
// split-K records (m, l) and o[128] of the calls that split. It is a static
// device array, so each GPU that loads the library holds its own copy until
// the process ends; the entry point allocates nothing. Host code never uses
// the name `scratch` as an address (on the host it only names the symbol):
// the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

struct nwd_ctx {
  nwd_desc desc;
  nwd::Shape shape;
  nwd::Workspace ws;
  int device;
  int forced_splits;
  int separate_merge;  // 1 separate kernel, 0 in the split kernel, -1 default (separate)
  int decode_kernel;   // -1 the launch's choice, 0 dot-product, 1 matrix-core
  int decode_layout;   // -1 the launch's choice, 0 contiguous key ranges, 1 strided blocks
  void* ev_start;      // hipEvent_t pair recorded around decode split kernels, or NULL
  void* ev_stop;
  int* status_host;    // pinned copy target of the device status word
  int64_t o_floats;    // floats allocated for ws.part_o
  void* q_pad;         // padded query / output rows of the padded-group decode
  void* out_pad;       //   and prefill (nwd::padded_group), or NULL
  int32_t* pos_sub;    // first positions of a padded prefill sub-chunk
  int pad_tokens;      // tokens of a padded prefill sub-chunk
  std::string err;
};

namespace {

thread_local std::string g_create_err;

// Workgroups one decode launch aims for: one 256-thread workgroup per CU
// (measured on MI355X, B = 1, per append + attend step: 32 splits, one
// workgroup per CU, 9.9-10.2 us at 4K against 11.8 / 11.1 / 12.2 / 12.3 for
// 16 / 24 / 40 / 48 splits, and 28.8-29.0 us at 32K against 42.9 / 30.9 /
// 36.1 / 32.2).
constexpr int kTargetWorkgroups = 256;
constexpr int kMinKeysPerSplit = 128;    // one workgroup iteration
constexpr int kMaxKeysPerSplit = 2048;   // bounds the slowest workgroup of a large batch
constexpr int kMaxSplits = 256;

int fail(nwd_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(nwd_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf;
  else g_create_err = buf;
  return code;
}

int hip_fail(nwd_ctx* ctx, const char* what, hipError_t e) {
  return fail(ctx, NWD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int resolve_len(const nwd_ctx* ctx, int32_t max_len) {
  return max_len <= 0 ? ctx->desc.max_seq : max_len;
}

// Split count for nwd_decode_attn. With few sequences (batch x query heads
// <= kSubSplitMaxWorkgroups) the decode runs one workgroup per query head
// and split; there one split (no merge launch) pays up to 384 keys, and
// n = kSubSplitMaxWorkgroups / (batch x heads) splits while they hold at
// most 256 keys each (up to 2048 keys at B = 1, 32 heads; per append +
// attend step at B = 1, 32 heads: 5.4 against 5.8 us at 320 keys, 5.8
// against 6.6 at 448, 6.1 against 8.1 with the per-KV-head form at 832,
// 7.0 against 8.2 at 1600, a tie at 2112, 12.2 against 10.1 at 4160).
// Otherwise one split up to 256 keys (6.5 against 7.9 us at 153 keys), and
// beyond, enough splits to fill the chip, even where that leaves splits with
// few keys (idle splits cost less than the unused CUs: 8.0-8.9 against
// 8.5-9.7 us per step from 384 to 2048 keys). Measured on MI355X.
//
// Past that, the split count keeps every workgroup of the launch in one
// wave of the chip (one per CU) while the sequences alone leave it at most
// half full (batch x KV heads <= 128): a partial second wave costs the whole
// per-split time again. B = 1, 32q/8kv, append + attend per step: 64K keys,
// 44.1 us with 32 splits (one wave) against 62.6 with 33 (the earlier
// 2048-key cap per split); 96K, 65.3 against 73.0 with 49; 128K, 83.5
// against 95.4 with 48 and 85.2 with 64 (two full waves). B = 2 at 32K, 43.7
// with 16 against 60.2 with 17; B = 4 at 32K, 82.4 with 8 against 95.0 with
// 17. Larger batches fill the chip by themselves and keep the 2048-key
// bound per split, which evens out ragged lengths (64 sequences of
// 512-16384 keys run 9 splits each).
int auto_splits(int n_heads, int n_kv_heads, int batch, int max_len) {
  const int units = (max_len + kMinKeysPerSplit - 1) / kMinKeysPerSplit;
  const int64_t heads = (int64_t)batch * n_heads;
  if (heads <= nwd::kSubSplitMaxWorkgroups) {
    if (units <= 3) return 1;
    const int n = (int)(nwd::kSubSplitMaxWorkgroups / heads);
    if (units <= 2 * n) return n;  // at most two 128-key units per split
  } else if (units <= 2) {
    return 1;
  }
  const int per_wave = batch * n_kv_heads;
  if (2 * per_wave <= kTargetWorkgroups) {  // one wave
    // A single sequence with splits of 1024-3072 keys runs faster on three
    // quarters of the wave: fewer merge records and less finishing-time skew,
    // with ~192 workgroups already at the read ceiling. Decode-only call,
    // 32q/8kv, 24 against 32 splits: 32K 24.05-24.13 against 24.31-24.55 us
    // (40q: 24.26-24.28 against 24.79-24.87), 64K 41.41-42.01 against
    // 42.04-42.87. Outside that range, or with more sequences, it loses:
    // 4K 9.09 against 8.72-8.75, 8K 11.75 against 10.92-11.03, 96K 65.2-65.4
    // against 64.0, 128K 84.3-84.4 against 83.4-83.5; B = 2 with 12 against
    // 16 splits, 16K 26.26 against 25.70, 32K 45.43 against 45.54 (a tie);
    // and with groups under 4 query heads (the dot-product kernel's shapes;
    // 32K: 8q 23.75-23.97 against 23.32-23.48, 16q 25.23-25.28 against
    // 24.05-24.08), while 64q gains as 32q does (24.48-24.59 against 24.98-25.0).
    const int n = kTargetWorkgroups / per_wave, n34 = 3 * n / 4;
    if (batch == 1 && n_heads >= 4 * n_kv_heads && n34 >= 1 && max_len >= 1024 * n34 &&
        max_len <= 3072 * n34)
      return n34;
    return n;
  }
  int n = (kTargetWorkgroups + per_wave - 1) / per_wave;              // fill the chip
  const int by_len = (max_len + kMaxKeysPerSplit - 1) / kMaxKeysPerSplit;  // bound per-split work
  if (by_len > n) n = by_len;
  return n < 1 ? 1 : n;
}

// At D = 128 and 64 every group up to 8 has split kernels and a prefill
// kernel built for it (groups 3, 6, 7: nwd_decode_groups.hip). At the other
// head sizes a group of 3, 6 or 7 runs the kernels of groups 4 / 8 on padded
// query rows (nwd_pad.hip), at every length: the two copy launches cost less
// than the general kernels' longer chains (decode calls on MI355X at D =
// 128, before those groups were built there, padded against general:
// 28q/4kv (group 7) 9.2 against 22.3 us at 1024 keys, 21.0 against 40.5 at
// 32768; 12q/2kv (group 6) 8.8 against 20.1 at 1024 keys; 24q/8kv (group
// 3) 10.0 against 14.0; built for the group: 6.1, 16.6, 5.9 and 6.3). The
// prefill of these groups runs the prefill kernels the same way. The
// allocation-free entry point, which has no padded buffers, uses the
// general kernels for them. Decode at head sizes 64 and 256 runs the
// dot-product split kernel built for them, and at the other multiples of 8
// up to 256 that kernel's padded form (groups 1, 2, 4, 5, and 8 up to 128;
// larger groups as several of those per KV head, nwd::kernel_group, or
// padded to one).
// Decode calls on MI355X, B = 1, against the general kernels: 32q/32kv/d96
// at 4096 keys 12.0 against 16.3 us, 32q/32kv/d80 11.6 against 15.0,
// 16q/8kv/d192 at 8192 keys 14.0 against 20.6, 64q/8kv/d120 15.5 against
// 30.3.
enum DecodeRoute { kRouteSpecialised = 0, kRoutePadded = 1, kRouteGeneral = 2 };

// The split kernels address a (sequence, KV head) slab with 32-bit byte
// offsets through buffer descriptors, so a slab may hold at most 1 GiB
// (head sizes above 128 with a longer max_seq take the general kernels).
bool slab_fits(const nwd::Shape& s) {
  return (int64_t)s.cap * s.head_dim * 2 <= ((int64_t)1 << 30);
}

DecodeRoute decode_route(const nwd::Shape& s, bool have_pad) {
  if (!slab_fits(s)) return kRouteGeneral;
  if (nwd::split_decode_shape(s.head_dim, s.group)) return kRouteSpecialised;
  if (have_pad && nwd::padded_decode_shape(s.head_dim, s.group)) return kRoutePadded;
  return kRouteGeneral;
}

// Prefill: the MFMA prefill kernels at head sizes 128 and 256 and the other
// multiples of 8 up to 256 (rows padded with zeros to 128 or 256 dims) with
// the groups nwd::kernel_group maps, and the others there through padded
// query rows; the general kernels otherwise. 512 tokens onto 8192 on MI355X,
// per call, against the general kernels: 32q/8kv/d64 77.6 against 1640 us,
// 32q/32kv/d96 79.1 against 7738, 16q/8kv/d256 80.7 against 3466.
DecodeRoute prefill_route(const nwd::Shape& s, bool have_pad) {
  if (!nwd::prefill_head_dim(s.head_dim) || !slab_fits(s)) return kRouteGeneral;
  int rep = 0;
  if (nwd::kernel_group(s.head_dim, s.group, &rep) > 0) return kRouteSpecialised;
  if (have_pad && nwd::padded_group(s.head_dim, s.group) > 0) return kRoutePadded;
  return kRouteGeneral;
}

// Whether a context of this shape gets the padded-row buffers.
bool wants_pad_buffers(int head_dim, int group) {
  return nwd::padded_group(head_dim, group) > 0 &&
         (nwd::padded_decode_shape(head_dim, group) || nwd::prefill_head_dim(head_dim));
}

// Workgroups per split of a decode on the split kernels: one per group of
// query heads the kernels run (nwd::kernel_group: kv_rep per KV head).
int kv_groups(const nwd::Shape& s) {
  int rep = 1;
  nwd::kernel_group(s.head_dim, s.group, &rep);
  return s.n_kv * rep;
}

int64_t general_units(const nwd::Shape& s, int batch, int n_new) {
  const int gp = nwd::general_heads_per_workgroup(s.head_dim, s.group);
  return (int64_t)batch * n_new * s.n_kv * ((s.group + gp - 1) / gp);
}

// Split count of the general-shape kernels (nwd_general.hip: one workgroup
// per split and `units` (sequence, query, KV head, head chunk)): about 512
// workgroups when the units alone are fewer, with at least 64 keys per split
// (one 16-key tile per wavefront). Decode calls on MI355X, us at 1/2x, 1x and
// 2x this count (bench.py --workload general, us_by_forced_splits):
// 16q/8kv/d256 at 8K keys 26.0 / 24.2 / 26.5 (64 splits), 32q/32kv/d96 at 4K
// 17.6 / 16.3 / 16.5 (16).
int general_splits(int64_t units, int max_len) {
  if (units >= 512) return 1;
  int n = (int)((512 + units - 1) / units);
  const int by_len = (max_len + 63) / 64;
  if (n > by_len) n = by_len;
  if (n > kMaxSplits) n = kMaxSplits;
  return n < 1 ? 1 : n;
}

// Validates a descriptor (the checks nwd_create and the allocation-free
// entry point share); failures name `who`.
int check_desc(const nwd_desc* d, const char* who) {
  if (!d) return fail(nullptr, NWD_ERR_INVALID, "%s: desc is NULL", who);
  if (d->n_heads <= 0 || d->n_kv_heads <= 0 || d->head_dim <= 0 || d->max_seq <= 0 ||
      d->max_batch <= 0)
    return fail(nullptr, NWD_ERR_INVALID,
                "%s: sizes must be positive (n_heads=%d n_kv_heads=%d head_dim=%d "
                "max_seq=%d max_batch=%d)",
                who, d->n_heads, d->n_kv_heads, d->head_dim, d->max_seq, d->max_batch);
  if (d->n_heads % d->n_kv_heads != 0)
    return fail(nullptr, NWD_ERR_INVALID, "%s: n_heads %d is not a multiple of n_kv_heads %d",
                who, d->n_heads, d->n_kv_heads);
  if (d->head_dim > nwd::kMaxHeadDim)
    return fail(nullptr, NWD_ERR_UNSUPPORTED, "%s: head_dim %d exceeds %d", who, d->head_dim,
                nwd::kMaxHeadDim);
  for (int t : {d->q_dtype, d->o_dtype, d->kv_dtype})
    if (t != NWD_F16 && t != NWD_F32)
      return fail(nullptr, NWD_ERR_INVALID, "%s: dtype %d is neither NWD_F16 nor NWD_F32", who, t);
  if (!(d->scale >= 0.f) || std::isinf(d->scale))
    return fail(nullptr, NWD_ERR_INVALID, "%s: scale must be finite and >= 0", who);
  if (d->max_seq > nwd::kMaxSeq)
    return fail(nullptr, NWD_ERR_UNSUPPORTED, "%s: max_seq %d exceeds %d tokens", who, d->max_seq,
                nwd::kMaxSeq);
  // Largest element index of a cache and of the query/output buffers must
  // fit the kernels' 64-bit index math; keep the per-slab token index in int.
  if ((int64_t)d->max_batch * d->n_kv_heads * (int64_t)d->max_seq > ((int64_t)1 << 40))
    return fail(nullptr, NWD_ERR_INVALID, "%s: cache too large", who);
  if ((int64_t)d->max_batch * d->n_kv_heads > (1 << 30))
    return fail(nullptr, NWD_ERR_INVALID, "%s: max_batch * n_kv_heads too large", who);
  return NWD_OK;
}

nwd::Shape shape_of(const nwd_desc* d) {
  nwd::Shape sh;
  sh.n_heads = d->n_heads;
  sh.n_kv = d->n_kv_heads;
  sh.group = d->n_heads / d->n_kv_heads;
  sh.cap = d->max_seq;
  sh.q16 = d->q_dtype == NWD_F16;
  sh.o16 = d->o_dtype == NWD_F16;
  sh.kv16 = d->kv_dtype == NWD_F16;
  sh.qk_scale = d->scale > 0.f ? d->scale : 1.0f / std::sqrt((float)d->head_dim);
  sh.head_dim = d->head_dim;
  return sh;
}

// Key layout over the splits (DecodeCall::layout). A batch of sequences
// takes the strided layout: the splits of a (sequence, KV head) then read
// neighbouring key blocks at any moment instead of batch x KV heads x splits
// separate streams (64 sequences of 512-16384 keys, append + attend, same
// box: 387.6-387.8 against 405.9-418.2 us per step). One sequence keeps
// contiguous ranges: there the strided layout tied at 32K keys (24.21-24.50
// against 24.33-24.43 us per append + attend step), lost at 64K keys with
// 24 splits (48.1-48.4 against 45.5-45.7) and at 1K keys (6.67 against
// 6.49), and gained only in decode-only calls at 4K-16K.
int default_layout(int batch, int max_len, int nsplit) {
  (void)max_len;
  return batch >= 2 && nsplit > 1 ? 1 : 0;
}

int clamp_splits(const nwd_ctx* ctx, const nwd::Shape& s, int batch, int n) {
  int cap = nwd::max_decode_splits(s, ctx->ws, batch);
  if (cap > kMaxSplits) cap = kMaxSplits;
  if (n > cap) n = cap;
  return n < 1 ? 1 : n;
}

// Records the static scratch holds for head size D: a 256-byte status
// slot, then (m, l) pairs and o[D] rows, each area 256-byte aligned.
constexpr size_t kScratchMlOffset = 256;
constexpr int64_t scratch_records(int D) { return (int64_t)(kScratchBytes - 512) / (8 + D * 4); }
constexpr size_t scratch_o_offset(int D) {
  return kScratchMlOffset + (size_t)((scratch_records(D) * 8 + 255) / 256) * 256;
}
constexpr bool scratch_fits(int D) {
  return scratch_o_offset(D) + (size_t)scratch_records(D) * D * 4 <= kScratchBytes;
}
static_assert(scratch_fits(1) && scratch_fits(nwd::kHeadDim) && scratch_fits(nwd::kMaxHeadDim),
              "records fit the scratch");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_dev[kMaxDevices];  // per device: the device address of `scratch`

// The device address of the current device's `scratch`, looked up on the
// first call on that device.
int scratch_address(const char* who, unsigned char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(nullptr, NWD_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(nullptr, NWD_ERR_UNSUPPORTED, "%s: device index %d beyond %d", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(nullptr, NWD_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", who,
                  hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<unsigned char*>(p);
  }
  *out = g_scratch_dev[dev];
  return NWD_OK;
}

}  // namespace

extern "C" {

int nwd_create(const nwd_desc* d, nwd_ctx** out_ctx) {
  if (!out_ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_create: out_ctx is NULL");
  *out_ctx = nullptr;
  if (int rc = check_desc(d, "nwd_create")) return rc;
  const int group = d->n_heads / d->n_kv_heads;
  // Split records of the kernels' width, and at least 128 floats per record:
  // the argmax records reuse part_o.
  const int o_dim = nwd::record_width(d->head_dim) > nwd::kHeadDim ? nwd::record_width(d->head_dim)
                                                                   : nwd::kHeadDim;

  nwd_ctx* ctx = new nwd_ctx();
  ctx->desc = *d;
  ctx->forced_splits = 0;
  ctx->separate_merge = -1;
  ctx->decode_kernel = -1;
  ctx->decode_layout = -1;
  ctx->ev_start = nullptr;
  ctx->ev_stop = nullptr;
  ctx->shape = shape_of(d);

  hipError_t e = hipGetDevice(&ctx->device);
  if (e != hipSuccess) {
    delete ctx;
    return fail(nullptr, NWD_ERR_HIP, "nwd_create: hipGetDevice: %s", hipGetErrorString(e));
  }
  // Split-K records: enough for kMaxSplits splits of one sequence, or
  // kTargetWorkgroups*2 workgroups' worth at max_batch.
  int64_t per_seq = (int64_t)d->n_heads * kMaxSplits;
  int64_t at_batch = (int64_t)group * 2 * kTargetWorkgroups;
  if ((int64_t)d->max_batch * d->n_heads > at_batch) at_batch = (int64_t)d->max_batch * d->n_heads;
  ctx->ws.records = per_seq > at_batch ? per_seq : at_batch;
  // Prefill splits a row tile's keys only while its row tiles underfill the
  // chip (< 256 tiles of 128 rows), so 2 * 256 * 128 records always suffice;
  // no more than the rows a call can have, times 2 splits.
  int64_t prefill = (int64_t)2 * d->max_seq * d->n_heads * d->max_batch;
  if (prefill > (int64_t)2 * kTargetWorkgroups * 128) prefill = (int64_t)2 * kTargetWorkgroups * 128;
  if (prefill > ctx->ws.records) ctx->ws.records = prefill;
  ctx->ws.part_o = nullptr;
  ctx->ws.part_ml = nullptr;
  ctx->q_pad = nullptr;
  ctx->out_pad = nullptr;
  ctx->pos_sub = nullptr;
  ctx->pad_tokens = 0;
  ctx->ws.status = nullptr;
  ctx->ws.counters = nullptr;
  ctx->status_host = nullptr;
  // Merge tickets: one per (sequence, group of query heads a workgroup
  // serves), at most one per (sequence, query head).
  size_t n_counters = (size_t)d->max_batch * d->n_heads;
  if (n_counters < (size_t)nwd::kSubSplitMaxWorkgroups) n_counters = nwd::kSubSplitMaxWorkgroups;
  ctx->o_floats = ctx->ws.records * o_dim;
  e = hipMalloc(&ctx->ws.part_o, ctx->o_floats * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&ctx->ws.part_ml, ctx->ws.records * sizeof(float2));
  if (e == hipSuccess) e = hipMalloc(&ctx->ws.counters, n_counters * sizeof(int));
  if (e == hipSuccess) e = hipMemset(ctx->ws.counters, 0, n_counters * sizeof(int));
  const int gp = nwd::padded_group(d->head_dim, group);
  if (e == hipSuccess && wants_pad_buffers(d->head_dim, group)) {
    // Padded rows of up to 512 prefill tokens per sub-chunk, within 32 MiB
    // per buffer (at least one token: the decode's rows).
    const size_t per_token = (size_t)d->max_batch * d->n_kv_heads * gp * d->head_dim * sizeof(float);
    size_t tokens = ((size_t)32 << 20) / per_token;
    if (tokens > 512) tokens = 512;
    if (tokens > (size_t)d->max_seq) tokens = (size_t)d->max_seq;
    if (tokens < 1) tokens = 1;
    ctx->pad_tokens = (int)tokens;
    e = hipMalloc(&ctx->q_pad, per_token * tokens);
    if (e == hipSuccess) e = hipMalloc(&ctx->out_pad, per_token * tokens);
    if (e == hipSuccess) e = hipMalloc(&ctx->pos_sub, (size_t)d->max_batch * sizeof(int32_t));
  }
  if (e == hipSuccess) e = hipMalloc(&ctx->ws.status, sizeof(int));
  if (e == hipSuccess) e = hipMemset(ctx->ws.status, 0, sizeof(int));
  // Pinned, so the per-step status read is one small DMA, not a staged copy.
  if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&ctx->status_host), sizeof(int));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    nwd_destroy(ctx);
    return fail(nullptr, NWD_ERR_HIP, "nwd_create: workspace allocation: %s", hipGetErrorString(e));
  }
  *out_ctx = ctx;
  return NWD_OK;
}

void nwd_destroy(nwd_ctx* ctx) {
  if (!ctx) return;
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(ctx->device);
  if (ctx->ws.part_o) (void)hipFree(ctx->ws.part_o);
  if (ctx->ws.part_ml) (void)hipFree(ctx->ws.part_ml);
  if (ctx->ws.counters) (void)hipFree(ctx->ws.counters);
  if (ctx->ws.status) (void)hipFree(ctx->ws.status);
  if (ctx->q_pad) (void)hipFree(ctx->q_pad);
  if (ctx->out_pad) (void)hipFree(ctx->out_pad);
  if (ctx->pos_sub) (void)hipFree(ctx->pos_sub);
  if (ctx->status_host) (void)hipHostFree(ctx->status_host);
  if (prev >= 0) (void)hipSetDevice(prev);
  delete ctx;
}

#ifndef NWD_SOURCE_HASH
#error "build with -DNWD_SOURCE_HASH=\"<sha256 of the sources>\" (build.py does)"
#endif
const char* nwd_source_hash(void) { return NWD_SOURCE_HASH; }

const char* nwd_last_error(const nwd_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

size_t nwd_cache_bytes(const nwd_ctx* ctx) {
  if (!ctx) return 0;
  return (size_t)ctx->desc.max_batch * ctx->desc.n_kv_heads * (size_t)ctx->desc.max_seq *
         ctx->desc.head_dim * 2;
}

int64_t nwd_cache_offset(const nwd_ctx* ctx, int32_t b, int32_t t, int32_t h, int32_t d) {
  if (!ctx || b < 0 || b >= ctx->desc.max_batch || t < 0 || t >= ctx->desc.max_seq || h < 0 ||
      h >= ctx->desc.n_kv_heads || d < 0 || d >= ctx->desc.head_dim)
    return -1;
  return nwd::cache_index_d(b, t, h, d, ctx->desc.n_kv_heads, ctx->desc.max_seq,
                            ctx->desc.head_dim);
}

int nwd_kv_append(nwd_ctx* ctx, const void* k_new, const void* v_new, void* k_cache,
                  void* v_cache, const int32_t* pos, int32_t batch, int32_t n_tokens,
                  void* stream) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_kv_append: ctx is NULL");
  if (!k_new || !v_new || !k_cache || !v_cache || !pos)
    return fail(ctx, NWD_ERR_INVALID, "nwd_kv_append: null buffer");
  if (batch < 1 || batch > ctx->desc.max_batch)
    return fail(ctx, NWD_ERR_CAPACITY, "nwd_kv_append: batch %d outside [1, max_batch=%d]", batch,
                ctx->desc.max_batch);
  if (n_tokens < 1 || n_tokens > ctx->desc.max_seq)
    return fail(ctx, NWD_ERR_CAPACITY, "nwd_kv_append: n_tokens %d outside [1, max_seq=%d]",
                n_tokens, ctx->desc.max_seq);
  hipError_t e = nwd::launch_kv_append(ctx->shape, k_new, v_new, k_cache, v_cache, pos, batch,
                                       n_tokens, ctx->ws.status, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_kv_append: launch", e);
  return NWD_OK;
}

int32_t nwd_decode_splits(const nwd_ctx* ctx, int32_t batch, int32_t max_len) {
  if (!ctx || batch < 1 || batch > ctx->desc.max_batch) return 0;
  int len = resolve_len(ctx, max_len);
  if (len > ctx->desc.max_seq) len = ctx->desc.max_seq;
  const DecodeRoute route = decode_route(ctx->shape, ctx->q_pad != nullptr);
  const nwd::Shape s = route == kRoutePadded ? nwd::padded_shape(ctx->shape) : ctx->shape;
  int n = ctx->forced_splits > 0 ? ctx->forced_splits
          : route == kRouteGeneral ? general_splits(general_units(s, batch, 1), len)
                                   : auto_splits(s.n_heads, kv_groups(s), batch, len);
  return clamp_splits(ctx, s, batch, n);
}

int nwd_set_decode_splits(nwd_ctx* ctx, int32_t n_splits) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_set_decode_splits: ctx is NULL");
  if (n_splits < 0) return fail(ctx, NWD_ERR_INVALID, "nwd_set_decode_splits: negative count");
  ctx->forced_splits = n_splits > kMaxSplits ? kMaxSplits : n_splits;
  return NWD_OK;
}

static int decode_common(nwd_ctx* ctx, const char* who, const void* q, const void* k_new,
                         const void* v_new, void* k_cache, void* v_cache, const int32_t* pos,
                         void* out, int32_t batch, int32_t max_len, void* stream) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "%s: ctx is NULL", who);
  if (!q || !k_cache || !v_cache || !pos || !out)
    return fail(ctx, NWD_ERR_INVALID, "%s: null buffer", who);
  if (batch < 1 || batch > ctx->desc.max_batch)
    return fail(ctx, NWD_ERR_CAPACITY, "%s: batch %d outside [1, max_batch=%d]", who, batch,
                ctx->desc.max_batch);
  const int len = resolve_len(ctx, max_len);
  if (len > ctx->desc.max_seq)
    return fail(ctx, NWD_ERR_CAPACITY, "%s: max_len %d exceeds max_seq %d", who, len,
                ctx->desc.max_seq);
  const DecodeRoute route = decode_route(ctx->shape, ctx->q_pad != nullptr);
  if (route == kRouteGeneral) {
    // General shapes: the append (if any) as its own launch, then the
    // general attention kernel and its merge.
    hipError_t e = hipSuccess;
    if (k_new)
      e = nwd::launch_kv_append(ctx->shape, k_new, v_new, k_cache, v_cache, pos, batch, 1,
                                ctx->ws.status, (hipStream_t)stream);
    if (e == hipSuccess)
      e = nwd::launch_general_attn(ctx->shape, q, k_cache, v_cache, pos, out, batch, 1, 0, len,
                                   nwd_decode_splits(ctx, batch, len), ctx->ws, ctx->ev_start,
                                   ctx->ev_stop, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(ctx, who, e);
    return NWD_OK;
  }
  nwd::DecodeCall c;
  c.q = q;
  c.k_cache = k_cache;
  c.v_cache = v_cache;
  c.pos = pos;
  c.out = out;
  c.k_new = k_new;
  c.v_new = v_new;
  c.batch = batch;
  c.nsplit = nwd_decode_splits(ctx, batch, len);
  c.span = len;
  // Default: the separate merge kernel, measured faster on MI355X at 4K and
  // 32K keys (its one launch costs less than the in-kernel merge's serialised
  // store, ticket and record round trips).
  c.fused_merge = ctx->separate_merge == 0 ? 1 : 0;
  c.kernel = ctx->decode_kernel;
  c.layout = ctx->decode_layout >= 0 ? ctx->decode_layout : default_layout(batch, len, c.nsplit);
  c.ev_start = ctx->ev_start;
  c.ev_stop = ctx->ev_stop;
  hipError_t e = route == kRoutePadded
                     ? nwd::launch_padded_decode(ctx->shape, c, ctx->ws, ctx->q_pad, ctx->out_pad,
                                                 (hipStream_t)stream)
                     : nwd::launch_decode(ctx->shape, c, ctx->ws, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, who, e);
  return NWD_OK;
}

int nwd_decode_attn(nwd_ctx* ctx, const void* q, const void* k_cache, const void* v_cache,
                    const int32_t* pos, void* out, int32_t batch, int32_t max_len,
                    void* stream) {
  return decode_common(ctx, "nwd_decode_attn", q, nullptr, nullptr, const_cast<void*>(k_cache),
                       const_cast<void*>(v_cache), pos, out, batch, max_len, stream);
}

int nwd_append_decode(nwd_ctx* ctx, const void* q, const void* k_new, const void* v_new,
                      void* k_cache, void* v_cache, const int32_t* pos, void* out,
                      int32_t batch, int32_t max_len, void* stream) {
  if (ctx && (!k_new || !v_new))
    return fail(ctx, NWD_ERR_INVALID, "nwd_append_decode: null new K/V rows");
  return decode_common(ctx, "nwd_append_decode", q, k_new, v_new, k_cache, v_cache, pos, out,
                       batch, max_len, stream);
}

int nwd_append_decode_noalloc(const nwd_desc* desc, const void* q, const void* k_new,
                              const void* v_new, void* k_cache, void* v_cache, const int32_t* pos,
                              void* out, int32_t batch, int32_t max_len, int32_t* status,
                              void* stream) {
  const char* who = "nwd_append_decode_noalloc";
  if (int rc = check_desc(desc, who)) return rc;
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !pos || !out)
    return fail(nullptr, NWD_ERR_INVALID, "%s: null buffer", who);
  if (batch < 1 || batch > desc->max_batch)
    return fail(nullptr, NWD_ERR_CAPACITY, "%s: batch %d outside [1, max_batch=%d]", who, batch,
                desc->max_batch);
  const int len = max_len <= 0 ? desc->max_seq : max_len;
  if (len > desc->max_seq)
    return fail(nullptr, NWD_ERR_CAPACITY, "%s: max_len %d exceeds max_seq %d", who, len,
                desc->max_seq);
  const nwd::Shape sh = shape_of(desc);
  const bool general = decode_route(sh, false) == kRouteGeneral;
  int n = general ? general_splits(general_units(sh, batch, 1), len)
                  : auto_splits(desc->n_heads, kv_groups(sh), batch, len);
  if (n > kMaxSplits) n = kMaxSplits;
  const int64_t records = n > 1 ? (int64_t)batch * desc->n_heads * n : 0;
  const int rw = nwd::record_width(desc->head_dim);  // floats per record
  const int64_t have = scratch_records(rw);
  if (records > have)
    return fail(nullptr, NWD_ERR_CAPACITY,
                "%s: %d sequences x %d heads x %d splits need %lld split records; the static "
                "scratch holds %lld at head_dim %d (%zu bytes)",
                who, batch, desc->n_heads, n, (long long)records, (long long)have,
                desc->head_dim, kScratchBytes);
  unsigned char* base = nullptr;
  if (int rc = scratch_address(who, &base)) return rc;
  nwd::Workspace ws;
  ws.part_ml = reinterpret_cast<float2*>(base + kScratchMlOffset);
  ws.part_o = reinterpret_cast<float*>(base + scratch_o_offset(rw));
  ws.records = have;
  ws.counters = nullptr;  // the separate merge kernel takes no arrival tickets
  ws.status = status ? status : reinterpret_cast<int*>(base);
  nwd::DecodeCall c;
  c.q = q;
  c.k_cache = k_cache;
  c.v_cache = v_cache;
  c.pos = pos;
  c.out = out;
  c.k_new = k_new;
  c.v_new = v_new;
  c.batch = batch;
  c.nsplit = n;
  c.span = len;
  c.fused_merge = 0;
  c.kernel = -1;
  c.layout = default_layout(batch, len, n);
  c.ev_start = nullptr;
  c.ev_stop = nullptr;
  hipError_t e = hipSuccess;
  if (general) {
    e = nwd::launch_kv_append(sh, k_new, v_new, k_cache, v_cache, pos, batch, 1, ws.status,
                              (hipStream_t)stream);
    if (e == hipSuccess)
      e = nwd::launch_general_attn(sh, q, k_cache, v_cache, pos, out, batch, 1, 0, len, n, ws,
                                   nullptr, nullptr, (hipStream_t)stream);
  } else {
    e = nwd::launch_decode(sh, c, ws, (hipStream_t)stream);
  }
  if (e != hipSuccess) return fail(nullptr, NWD_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
  return NWD_OK;
}

int nwd_set_decode_merge(nwd_ctx* ctx, int32_t separate_kernel) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_set_decode_merge: ctx is NULL");
  ctx->separate_merge = separate_kernel < 0 ? -1 : (separate_kernel ? 1 : 0);
  return NWD_OK;
}

int nwd_set_decode_kernel(nwd_ctx* ctx, int32_t kernel) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_set_decode_kernel: ctx is NULL");
  if (kernel < -1 || kernel > 1)
    return fail(ctx, NWD_ERR_INVALID, "nwd_set_decode_kernel: kernel %d is not -1, 0 or 1", kernel);
  ctx->decode_kernel = kernel;
  return NWD_OK;
}

int nwd_set_decode_layout(nwd_ctx* ctx, int32_t layout) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_set_decode_layout: ctx is NULL");
  if (layout < -1 || layout > 1)
    return fail(ctx, NWD_ERR_INVALID, "nwd_set_decode_layout: layout %d is not -1, 0 or 1", layout);
  ctx->decode_layout = layout;
  return NWD_OK;
}

int nwd_set_kernel_events(nwd_ctx* ctx, void* start_event, void* stop_event) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_set_kernel_events: ctx is NULL");
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(ctx, NWD_ERR_INVALID, "nwd_set_kernel_events: give both events or neither");
  ctx->ev_start = start_event;
  ctx->ev_stop = stop_event;
  return NWD_OK;
}

int nwd_prefill_attn(nwd_ctx* ctx, const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* pos0, void* out, int32_t batch, int32_t n_new,
                     int32_t max_len, void* stream) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_prefill_attn: ctx is NULL");
  if (!q || !k_cache || !v_cache || !pos0 || !out)
    return fail(ctx, NWD_ERR_INVALID, "nwd_prefill_attn: null buffer");
  if (batch < 1 || batch > ctx->desc.max_batch)
    return fail(ctx, NWD_ERR_CAPACITY, "nwd_prefill_attn: batch %d outside [1, max_batch=%d]",
                batch, ctx->desc.max_batch);
  if (n_new < 1 || n_new > ctx->desc.max_seq)
    return fail(ctx, NWD_ERR_CAPACITY, "nwd_prefill_attn: n_new %d outside [1, max_seq=%d]", n_new,
                ctx->desc.max_seq);
  const int len = resolve_len(ctx, max_len);
  if (len > ctx->desc.max_seq || len < n_new)
    return fail(ctx, NWD_ERR_CAPACITY, "nwd_prefill_attn: max_len %d outside [n_new, max_seq=%d]",
                len, ctx->desc.max_seq);
  hipError_t e;
  const DecodeRoute route = prefill_route(ctx->shape, ctx->q_pad != nullptr);
  if (route == kRoutePadded) {
    nwd::PadBuffers pb{ctx->q_pad, ctx->out_pad, ctx->pos_sub, ctx->pad_tokens};
    e = nwd::launch_padded_prefill(ctx->shape, q, k_cache, v_cache, pos0, out, batch, n_new, len,
                                   ctx->ws, pb, (hipStream_t)stream);
  } else if (route == kRouteGeneral) {
    const int64_t rows = (int64_t)batch * n_new * ctx->desc.n_heads;
    if (rows > 0x7FFFFFFF)
      return fail(ctx, NWD_ERR_CAPACITY, "nwd_prefill_attn: %lld output rows exceed 2^31 - 1",
                  (long long)rows);
    int n = ctx->forced_splits > 0 ? ctx->forced_splits
                                   : general_splits(general_units(ctx->shape, batch, n_new), len);
    const int64_t fit = ctx->ws.records / rows;
    if (n > fit) n = (int)fit;
    if (n < 1) n = 1;
    e = nwd::launch_general_attn(ctx->shape, q, k_cache, v_cache, pos0, out, batch, n_new, 1, len,
                                 n, ctx->ws, nullptr, nullptr, (hipStream_t)stream);
  } else {
    e = nwd::launch_prefill(ctx->shape, q, k_cache, v_cache, pos0, out, batch, n_new, len,
                            ctx->ws, (hipStream_t)stream);
  }
  if (e == hipErrorNotSupported)
    return fail(ctx, NWD_ERR_UNSUPPORTED, "nwd_prefill_attn: this shape is not built");
  if (e != hipSuccess) return hip_fail(ctx, "nwd_prefill_attn: launch", e);
  return NWD_OK;
}

int nwd_device_status(nwd_ctx* ctx, void* stream) {
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "nwd_device_status: ctx is NULL");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(ctx->status_host, ctx->ws.status, sizeof(int), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_device_status", e);
  const int host = *ctx->status_host;
  if (host == 0) return NWD_OK;
  e = hipMemsetAsync(ctx->ws.status, 0, sizeof(int), s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_device_status: clear", e);
  if (host & nwd::kStatusOutOfBounds)
    return fail(ctx, NWD_ERR_DEVICE,
                "a kernel of this bounds-checked build computed an address outside its "
                "buffer; the access was skipped (status bits 0x%x)",
                host);
  if (host & nwd::kStatusQueryRange)
    return fail(ctx, NWD_ERR_DEVICE,
                "a query element left the fp16 range of the matrix-core kernels (prefill: "
                "|q| * scale * log2(e) > 65504; decode with fp32 queries: |q| > 65504): "
                "those outputs are not finite (status bits 0x%x)",
                host);
  return fail(ctx, NWD_ERR_DEVICE,
              "a kernel saw a position outside [0, max_seq=%d): the cache was not written "
              "there and attention was clamped to the capacity",
              ctx->desc.max_seq);
}

// Checks one 4-bit projection descriptor; `cols` > 0 also fixes its width.
static int check_q4(nwd_ctx* ctx, const char* who, const char* name, const nwd_q4_weight* w,
                    int cols) {
  if (!w) return fail(ctx, NWD_ERR_INVALID, "%s: %s is NULL", who, name);
  if (!w->quant || !w->scales || !w->zp)
    return fail(ctx, NWD_ERR_INVALID, "%s: %s has a null buffer", who, name);
  if (reinterpret_cast<uintptr_t>(w->quant) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(w->scales) % 4 != 0)
    return fail(ctx, NWD_ERR_INVALID, "%s: %s quant must be 16-byte and scales 4-byte aligned",
                who, name);
  if (w->n < 1 || (cols > 0 && w->n != cols))
    return fail(ctx, NWD_ERR_INVALID, "%s: %s has %d columns, expected %d", who, name, w->n,
                cols > 0 ? cols : 1);
  if (w->n_blocks < 1 || w->n_blocks > nwd::kQ4MaxBlocks)
    return fail(ctx, NWD_ERR_UNSUPPORTED, "%s: %s n_blocks %d outside [1, %d] (K <= %d)", who,
                name, w->n_blocks, nwd::kQ4MaxBlocks, 32 * nwd::kQ4MaxBlocks);
  return NWD_OK;
}

static nwd::Q4Mat q4_mat(const nwd_q4_weight* w) {
  return nwd::Q4Mat{static_cast<const uint8_t*>(w->quant), w->scales,
                    static_cast<const uint8_t*>(w->zp), w->n};
}

int nwd_q4_gemv(nwd_ctx* ctx, const float* a, const nwd_q4_weight* w, float* y, int32_t batch,
                int32_t epilogue, void* stream) {
  const char* who = "nwd_q4_gemv";
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "%s: ctx is NULL", who);
  if (int rc = check_q4(ctx, who, "w", w, 0)) return rc;
  if (!a || !y) return fail(ctx, NWD_ERR_INVALID, "%s: null buffer", who);
  if (reinterpret_cast<uintptr_t>(a) % 16 != 0 || reinterpret_cast<uintptr_t>(y) % 4 != 0)
    return fail(ctx, NWD_ERR_INVALID, "%s: a must be 16-byte and y 4-byte aligned", who);
  if (batch < 1 || batch > 65535)
    return fail(ctx, NWD_ERR_INVALID, "%s: batch %d outside [1, 65535]", who, batch);
  if (epilogue != NWD_Q4_PLAIN && epilogue != NWD_Q4_RELU2 && epilogue != NWD_Q4_ACCUMULATE)
    return fail(ctx, NWD_ERR_INVALID, "%s: unknown epilogue %d", who, epilogue);
  hipError_t e = nwd::launch_q4_gemv(a, q4_mat(w), w->n_blocks, y, batch, epilogue,
                                     (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_q4_gemv: launch", e);
  return NWD_OK;
}

int nwd_qkv_append(nwd_ctx* ctx, const float* x, const nwd_q4_weight* wq, const nwd_q4_weight* wk,
                   const nwd_q4_weight* wv, void* q_out, void* k_cache, void* v_cache,
                   const int32_t* pos, int32_t batch, void* stream) {
  const char* who = "nwd_qkv_append";
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "%s: ctx is NULL", who);
  const int dq = ctx->desc.n_heads * ctx->desc.head_dim;
  const int dkv = ctx->desc.n_kv_heads * ctx->desc.head_dim;
  if (int rc = check_q4(ctx, who, "wq", wq, dq)) return rc;
  if (int rc = check_q4(ctx, who, "wk", wk, dkv)) return rc;
  if (int rc = check_q4(ctx, who, "wv", wv, dkv)) return rc;
  if (wk->n_blocks != wq->n_blocks || wv->n_blocks != wq->n_blocks)
    return fail(ctx, NWD_ERR_INVALID, "%s: wq, wk and wv must share K (n_blocks %d, %d, %d)", who,
                wq->n_blocks, wk->n_blocks, wv->n_blocks);
  if (!x || !q_out || !k_cache || !v_cache || !pos)
    return fail(ctx, NWD_ERR_INVALID, "%s: null buffer", who);
  // A workgroup's 16 columns must lie in one of the q, k, v ranges and a
  // wavefront's 4 in one head.
  if (ctx->desc.head_dim % 4 != 0 || dq % 16 != 0 || dkv % 16 != 0)
    return fail(ctx, NWD_ERR_UNSUPPORTED,
                "%s: head_dim %d needs n_heads * head_dim and n_kv_heads * head_dim to be "
                "multiples of 16 and head_dim a multiple of 4",
                who, ctx->desc.head_dim);
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(q_out) % 16 != 0)
    return fail(ctx, NWD_ERR_INVALID, "%s: x and q_out must be 16-byte aligned", who);
  if (batch < 1 || batch > ctx->desc.max_batch)
    return fail(ctx, NWD_ERR_CAPACITY, "%s: batch %d outside [1, max_batch=%d]", who, batch,
                ctx->desc.max_batch);
  hipError_t e = nwd::launch_qkv_append(ctx->shape, x, q4_mat(wq), q4_mat(wk), q4_mat(wv),
                                        wq->n_blocks, q_out, k_cache, v_cache, pos, batch,
                                        ctx->ws.status, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_qkv_append: launch", e);
  return NWD_OK;
}

// The argmax records live in the split-K workspace (calls on a context are
// stream-ordered, so they never overlap a decode's use of it).
static unsigned long long* argmax_records(nwd_ctx* ctx, const char* who, int64_t count, int* rc) {
  const int64_t have = ctx->o_floats * (int64_t)sizeof(float) / 8;
  if (count > have) {
    *rc = fail(ctx, NWD_ERR_CAPACITY, "%s: %lld partial records exceed the workspace (%lld)", who,
               (long long)count, (long long)have);
    return nullptr;
  }
  *rc = NWD_OK;
  return reinterpret_cast<unsigned long long*>(ctx->ws.part_o);
}

int nwd_argmax(nwd_ctx* ctx, const float* x, int32_t n, uint32_t* out, int32_t batch,
               void* stream) {
  const char* who = "nwd_argmax";
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "%s: ctx is NULL", who);
  if (!x || !out) return fail(ctx, NWD_ERR_INVALID, "%s: null buffer", who);
  if (n < 1) return fail(ctx, NWD_ERR_INVALID, "%s: n %d < 1", who, n);
  if (batch < 1 || batch > 65535)
    return fail(ctx, NWD_ERR_INVALID, "%s: batch %d outside [1, 65535]", who, batch);
  int rc;
  unsigned long long* rec =
      argmax_records(ctx, who, (int64_t)nwd::argmax_records_per_row(n) * batch, &rc);
  if (!rec) return rc;
  hipError_t e = nwd::launch_argmax(x, n, out, batch, rec, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_argmax: launch", e);
  return NWD_OK;
}

int nwd_lm_head_argmax(nwd_ctx* ctx, const float* h, const nwd_q4_weight* w, float* logits,
                       uint32_t* out, int32_t batch, void* stream) {
  const char* who = "nwd_lm_head_argmax";
  if (!ctx) return fail(nullptr, NWD_ERR_INVALID, "%s: ctx is NULL", who);
  if (int r = check_q4(ctx, who, "w", w, 0)) return r;
  if (!h || !out) return fail(ctx, NWD_ERR_INVALID, "%s: null buffer", who);
  if (reinterpret_cast<uintptr_t>(h) % 16 != 0)
    return fail(ctx, NWD_ERR_INVALID, "%s: h must be 16-byte aligned", who);
  if (batch < 1 || batch > 65535)
    return fail(ctx, NWD_ERR_INVALID, "%s: batch %d outside [1, 65535]", who, batch);
  int rc;
  unsigned long long* rec =
      argmax_records(ctx, who, (int64_t)nwd::q4_argmax_records_per_row(w->n) * batch, &rc);
  if (!rec) return rc;
  hipError_t e = nwd::launch_q4_argmax(h, q4_mat(w), w->n_blocks, logits, out, batch, rec,
                                       (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, "nwd_lm_head_argmax: launch", e);
  return NWD_OK;
}

}  // extern "C"
