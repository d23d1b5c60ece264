// nwd_decode.hip — decode GQA attention for gfx950 (split-K + merge).
//
// Replaces kernels/sparse_attn.wgsl main (:31-114). The reference runs one
// 64-thread workgroup per QUERY head (engine/runtime.js:391), so each of the
// G = H/Hkv query heads of a group re-reads the same K/V rows, with one
// thread streaming one whole key row (uncoalesced), and it caps the context
// at 256 keys (:29).
//
// Here one workgroup owns (sequence b, KV head hkv, split s): it loads each
// K/V row of its key range once and serves all G query heads of the group
// from it. When few sequences leave the chip nearly idle, the launch instead
// gives each query head its own workgroups (kQsub = G workgroups per KV head,
// each serving one head), which shortens every workgroup's serial chain
// G-fold.
//
// Mapping inside a wavefront: rows of kLanes lanes (16 or 8); a row owns one
// key at a time and each lane holds 128 / kLanes of its dims (one or two
// 16-byte runs), so one load instruction reads 1 KB of consecutive keys. q.k
// is a packed fp16 dot (v_dot2_f32_f16) or an fp32 FMA chain, summed over the
// row's lanes with DPP moves, so every lane of the row holds the score. Each
// row runs its own online softmax (running max and sum in log2 units, exp2
// on the hardware) and accumulates p * V for its dims in fp32 with no
// cross-lane traffic. The next iteration's K/V loads are issued before the
// current one is computed, unconditionally, so the wait before the compute
// only waits for the older loads; they go through buffer descriptors that
// end at the split's last key, so the prefetch past the end reads zeros
// without a memory round trip, and they are marked non-temporal (each byte
// is read once). At the end the row states are merged (DPP and lane swaps
// inside a wave, LDS across waves) into one record (m, l, o[128]) per query
// head.
//
// With one split the record is normalised and written to `out`. With
// several, records go to the workspace and decode_merge_kernel combines them
// — the partial/merge structure of kernels/argmax_partial.wgsl:16-52 and
// kernels/argmax_merge.wgsl:8-42, with (max, sum, o[D]) records instead of
// (value, index) pairs. Optionally (nwd_set_decode_merge) the merge runs in
// the split kernel itself: records are written through to memory (vector
// stores with the agent-coherent cache policy sc1) and the workgroup that
// takes the last arrival ticket of its (b, hkv) reads them with sc1 loads
// and merges them.
//
// The key range is partitioned from the host's length bound (max_len), not
// from the device position, so a workgroup's first K/V loads do not wait for
// the position load; the position only masks keys and bounds the loop, and
// the last split extends past the bound if the position exceeds it.
//
// Fused append: when new K/V rows are given, the workgroup whose range holds
// the new position writes them into the caches and uses them from registers,
// so an attention-layer step (kv_append x2 + attention in the reference,
// engine/runtime.js:389-391) is one launch.
#include "nwd_decode_mfma.h"

namespace nwd {

// Groups built as they are: 1, 2, 4, 5 and 8 (8 up to head size 128), at
// head sizes 128 and 64 every group up to 8, and 3 at 256 (3, 6 and 7 in
// nwd_decode_groups.hip). A larger group runs as groups of a built size, so
// that each KV head's rows are read as few times as possible: kv_rep =
// ceil(group / largest) reads. A built divisor (the largest first) that
// gives that many groups takes the group as it is; otherwise it is padded
// to a multiple of the largest size. Decode calls on MI355X, B = 1, 8192
// keys: 96q/8kv/d128 (group 12) as 3 groups of 4, 20.6 us, padded to 16 as
// 2 groups of 8, 16.5, as 2 groups of 6, 12.2 (128q/8kv, 2 groups of 8:
// 12.4; on the general kernels 43.3).
int kernel_group(int head_dim, int group, int* kv_rep) {
  *kv_rep = 1;
  const bool every = head_dim == kHeadDim || head_dim == 64;  // 1 .. 8 all built
  const int top = head_dim <= kHeadDim ? 8 : 5;  // group 8 is built up to head size 128
  auto built = [&](int g) {
    return g == 1 || g == 2 || g == 4 || g == 5 || g == top || (every && g >= 3 && g <= 8) ||
           (head_dim == 256 && g == 3);
  };
  if (built(group)) return group;
  if (group <= top) return 0;  // 3, 6, 7 at other head sizes: padded first
  const int reads = (group + top - 1) / top;
  for (int gs = top; gs >= 3; --gs) {
    if (built(gs) && group % gs == 0 && group / gs == reads) {
      *kv_rep = reads;
      return gs;
    }
  }
  return 0;
}

int padded_group(int head_dim, int group) {
  int rep = 0;
  if (kernel_group(head_dim, group, &rep) > 0) return 0;
  if (group == 3) return 4;
  if (group < 8) return 8;
  const int top = head_dim <= kHeadDim ? 8 : 5;
  return (group + top - 1) / top * top;
}

bool split_decode_shape(int head_dim, int group) {
  int rep = 0;
  return head_dim >= 8 && head_dim <= 256 && head_dim % 8 == 0 &&
         kernel_group(head_dim, group, &rep) > 0;
}

hipError_t launch_decode(const Shape& s0, const DecodeCall& c, const Workspace& ws,
                         hipStream_t stream) {
  if (!split_decode_shape(s0.head_dim, s0.group)) return hipErrorInvalidValue;
  // A group the kernels are not built for runs as kv_rep groups of a built
  // size per KV head (kernel_group); the kernels then see n_kv * kv_rep KV
  // heads of that group.
  int kv_rep = 1;
  Shape s = s0;
  s.group = kernel_group(s0.head_dim, s0.group, &kv_rep);
  s.n_kv = s0.n_kv * kv_rep;
  DecodeArgs a;
  a.q = c.q;
  a.k_cache = static_cast<f16*>(c.k_cache);
  a.v_cache = static_cast<f16*>(c.v_cache);
  a.pos = c.pos;
  a.out = c.out;
  a.part_o = ws.part_o;
  a.part_ml = ws.part_ml;
  a.records = ws.records;
  a.k_new = c.k_new;
  a.v_new = c.v_new;
  a.new16 = s.kv16;
  a.batch = c.batch;
  a.n_heads = s.n_heads;
  a.n_kv = s.n_kv;
  a.cap = s.cap;
  a.nsplit = c.nsplit;
  a.span = c.span;
  a.counters = ws.counters;
  a.fused_merge = c.fused_merge;
  a.strided = c.layout == 1;
  a.qk_scale_log2 = s.qk_scale * kLog2e;
  a.status = ws.status;
  a.head_dim = s.head_dim;
  a.kv_rep = kv_rep;
  if (s.head_dim != kHeadDim) return launch_decode_other(s, a, c, stream);
  switch (s.group) {
    case 1: return launch_decode_128<1>(s, a, c, stream);
    case 2: return launch_decode_128<2>(s, a, c, stream);
    case 4: return launch_decode_128<4>(s, a, c, stream);
    case 5: return launch_decode_128<5>(s, a, c, stream);
    case 8: return launch_decode_128<8>(s, a, c, stream);
    default: return launch_decode_groups(s, a, c, stream);  // 3, 6, 7
  }
}

int max_decode_splits(const Shape& s, const Workspace& ws, int batch) {
  const int64_t per = (int64_t)batch * s.n_heads;
  int64_t m = per > 0 ? ws.records / per : 0;
  if (m > 256) m = 256;
  return (int)m;
}

}  // namespace nwd
