// Host driver for the AddressSanitizer build of libnwd_attn.so: drives the C
// ABI (include/nwd_attn.h) so that ASan checks the library's host code: the
// argument validation and error formatting, the context's allocations and
// release, and the launch set-up of every entry point. Device code is built
// as in the product library; GPU memory is not checked here.
//
//   nwd_abi_asan cpu   validation paths only: no HIP runtime call is made
//   nwd_abi_asan gpu   also, per query-head group, one context through every
//                      entry point with buffers of exactly the documented
//                      sizes, then released (needs a GPU)
//
// Prints one line per phase and exits 0 when every call returned what it
// should; an ASan report aborts the program with a non-zero status.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "nwd_attn.h"

static int g_calls = 0, g_failed = 0;

static void expect(int got, int want, const char* what, const nwd_ctx* ctx) {
  ++g_calls;
  if (got == want) return;
  ++g_failed;
  std::fprintf(stderr, "FAIL %s: returned %d, expected %d (%s)\n", what, got, want,
               nwd_last_error(ctx));
}

static nwd_desc make_desc(int h, int hkv, int max_seq, int max_batch) {
  nwd_desc d;
  std::memset(&d, 0, sizeof d);
  d.n_heads = h;
  d.n_kv_heads = hkv;
  d.head_dim = 128;
  d.max_seq = max_seq;
  d.max_batch = max_batch;
  d.q_dtype = NWD_F16;
  d.o_dtype = NWD_F16;
  d.kv_dtype = NWD_F16;
  d.scale = 0.f;
  return d;
}

// Every rejection nwd_create makes before it touches the GPU, then the null
// context and null argument paths of each entry point.
static void cpu_checks() {
  struct Bad {
    int field, value, want;
  };
  const Bad bad[] = {
      {0, 0, NWD_ERR_INVALID},           {1, -1, NWD_ERR_INVALID},
      {0, 30, NWD_ERR_INVALID},          {2, 0, NWD_ERR_INVALID},
      {2, 513, NWD_ERR_UNSUPPORTED},
      {3, 0, NWD_ERR_INVALID},           {3, (1 << 22) + 1, NWD_ERR_UNSUPPORTED},
      {4, 0, NWD_ERR_INVALID},           {5, 7, NWD_ERR_INVALID},
  };
  for (const Bad& b : bad) {
    nwd_desc d = make_desc(32, 8, 4096, 1);
    int32_t* f[] = {&d.n_heads, &d.n_kv_heads, &d.head_dim, &d.max_seq, &d.max_batch, &d.q_dtype};
    *f[b.field] = b.value;
    nwd_ctx* ctx = reinterpret_cast<nwd_ctx*>(0x1234);
    expect(nwd_create(&d, &ctx), b.want, "nwd_create(bad descriptor)", nullptr);
    if (ctx != nullptr) {
      ++g_failed;
      std::fprintf(stderr, "FAIL nwd_create left a context on failure\n");
    }
    if (std::strncmp(nwd_last_error(nullptr), "nwd_create", 10) != 0) {
      ++g_failed;
      std::fprintf(stderr, "FAIL nwd_create error text: %s\n", nwd_last_error(nullptr));
    }
  }
  for (float s : {-1.f, NAN, INFINITY}) {
    nwd_desc d = make_desc(32, 8, 4096, 1);
    d.scale = s;
    nwd_ctx* ctx = nullptr;
    expect(nwd_create(&d, &ctx), NWD_ERR_INVALID, "nwd_create(bad scale)", nullptr);
  }
  expect(nwd_create(nullptr, nullptr), NWD_ERR_INVALID, "nwd_create(NULL)", nullptr);
  nwd_ctx* none = nullptr;
  expect(nwd_create(nullptr, &none), NWD_ERR_INVALID, "nwd_create(NULL desc)", nullptr);
  expect(nwd_kv_append(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1, nullptr),
         NWD_ERR_INVALID, "nwd_kv_append(NULL)", nullptr);
  expect(nwd_decode_attn(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 0, nullptr),
         NWD_ERR_INVALID, "nwd_decode_attn(NULL)", nullptr);
  expect(nwd_append_decode(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           1, 0, nullptr),
         NWD_ERR_INVALID, "nwd_append_decode(NULL)", nullptr);
  expect(nwd_prefill_attn(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1, 0, nullptr),
         NWD_ERR_INVALID, "nwd_prefill_attn(NULL)", nullptr);
  expect(nwd_device_status(nullptr, nullptr), NWD_ERR_INVALID, "nwd_device_status(NULL)", nullptr);
  expect(nwd_set_decode_splits(nullptr, 3), NWD_ERR_INVALID, "nwd_set_decode_splits(NULL)",
         nullptr);
  expect(nwd_set_decode_merge(nullptr, 1), NWD_ERR_INVALID, "nwd_set_decode_merge(NULL)", nullptr);
  expect(nwd_set_decode_kernel(nullptr, 1), NWD_ERR_INVALID, "nwd_set_decode_kernel(NULL)", nullptr);
  expect(nwd_set_kernel_events(nullptr, nullptr, nullptr), NWD_ERR_INVALID,
         "nwd_set_kernel_events(NULL)", nullptr);
  expect(nwd_q4_gemv(nullptr, nullptr, nullptr, nullptr, 1, 0, nullptr), NWD_ERR_INVALID,
         "nwd_q4_gemv(NULL)", nullptr);
  expect(nwd_qkv_append(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                        nullptr, 1, nullptr),
         NWD_ERR_INVALID, "nwd_qkv_append(NULL)", nullptr);
  expect(nwd_argmax(nullptr, nullptr, 1, nullptr, 1, nullptr), NWD_ERR_INVALID,
         "nwd_argmax(NULL)", nullptr);
  expect(nwd_lm_head_argmax(nullptr, nullptr, nullptr, nullptr, nullptr, 1, nullptr),
         NWD_ERR_INVALID, "nwd_lm_head_argmax(NULL)", nullptr);
  // the allocation-free entry point validates its descriptor on the host
  nwd_desc d = make_desc(32, 8, 4096, 1);
  d.head_dim = 513;
  expect(nwd_append_decode_noalloc(&d, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                   nullptr, 1, 0, nullptr, nullptr),
         NWD_ERR_UNSUPPORTED, "nwd_append_decode_noalloc(head_dim 513)", nullptr);
  expect(nwd_append_decode_noalloc(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                   nullptr, 1, 0, nullptr, nullptr),
         NWD_ERR_INVALID, "nwd_append_decode_noalloc(NULL)", nullptr);
  if (nwd_cache_bytes(nullptr) != 0 || nwd_cache_offset(nullptr, 0, 0, 0, 0) != -1 ||
      nwd_decode_splits(nullptr, 1, 100) != 0) {
    ++g_failed;
    std::fprintf(stderr, "FAIL NULL-context queries\n");
  }
  g_calls += 3;
  nwd_destroy(nullptr);
}

// Device allocations of exactly `bytes`, released together.
struct DevBufs {
  std::vector<void*> ptrs;
  void* get(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess || hipMemset(p, 0, bytes) != hipSuccess) {
      std::fprintf(stderr, "FAIL hipMalloc(%zu)\n", bytes);
      std::exit(3);
    }
    ptrs.push_back(p);
    return p;
  }
  ~DevBufs() {
    for (void* p : ptrs) (void)hipFree(p);
  }
};

struct Q4 {
  nwd_q4_weight w;
  Q4(DevBufs& m, int n, int n_blocks) {
    w.quant = m.get((size_t)n * n_blocks * 16);
    w.scales = static_cast<const float*>(m.get((size_t)n * n_blocks * sizeof(float)));
    w.zp = m.get(((size_t)n * n_blocks + 1) / 2);
    w.n = n;
    w.n_blocks = n_blocks;
  }
};

// One context of group g and head size d through every entry point: batch
// 2, 512 positions (d = 128 runs the kernels built for each group up to 8,
// groups 4 and 7 at d = 64 and group 5 at d = 256 the decode split kernel
// built for those sizes and the MFMA prefills, group 3 at d = 96 and group 7
// at d = 80 the padded-group route, group 12 at d = 96 padded to two groups
// of 8 per KV head on the padded head-size forms, group 2 at d = 100 the
// general kernels).
static void gpu_cycle(int group, int d) {
  const int hkv = 8, h = hkv * group, batch = 2, max_seq = 512;
  nwd_desc desc = make_desc(h, hkv, max_seq, batch);
  desc.head_dim = d;
  nwd_ctx* ctx = nullptr;
  expect(nwd_create(&desc, &ctx), NWD_OK, "nwd_create", nullptr);
  if (!ctx) return;
  {
    DevBufs m;
    const size_t cache = nwd_cache_bytes(ctx);
    if (cache != (size_t)batch * hkv * max_seq * d * 2) {  // the buffers below assume it
      ++g_failed;
      std::fprintf(stderr, "FAIL nwd_cache_bytes %zu: no kernel launched\n", cache);
      m.ptrs.clear();
      nwd_destroy(ctx);
      return;
    }
    void* kc = m.get(cache);
    void* vc = m.get(cache);
    void* q = m.get((size_t)batch * h * d * 2);
    void* out = m.get((size_t)batch * h * d * 2);
    void* kn = m.get((size_t)batch * hkv * d * 2);
    void* vn = m.get((size_t)batch * hkv * d * 2);
    const int32_t pos_h[batch] = {10, 300};
    auto* pos = static_cast<int32_t*>(m.get(sizeof pos_h));
    (void)hipMemcpy(pos, pos_h, sizeof pos_h, hipMemcpyHostToDevice);
    expect(nwd_kv_append(ctx, kn, vn, kc, vc, pos, batch, 1, nullptr), NWD_OK, "nwd_kv_append",
           ctx);
    expect(nwd_decode_attn(ctx, q, kc, vc, pos, out, batch, 0, nullptr), NWD_OK,
           "nwd_decode_attn", ctx);
    expect(nwd_append_decode(ctx, q, kn, vn, kc, vc, pos, out, batch, 0, nullptr), NWD_OK,
           "nwd_append_decode", ctx);
    expect(nwd_set_decode_splits(ctx, 3), NWD_OK, "nwd_set_decode_splits(3)", ctx);
    expect(nwd_set_decode_merge(ctx, 1), NWD_OK, "nwd_set_decode_merge(1)", ctx);
    expect(nwd_decode_attn(ctx, q, kc, vc, pos, out, batch, 0, nullptr), NWD_OK,
           "nwd_decode_attn(3 splits)", ctx);
    expect(nwd_set_decode_splits(ctx, 0), NWD_OK, "nwd_set_decode_splits(0)", ctx);
    expect(nwd_set_decode_merge(ctx, -1), NWD_OK, "nwd_set_decode_merge(-1)", ctx);
    expect(nwd_set_decode_kernel(ctx, 2), NWD_ERR_INVALID, "nwd_set_decode_kernel(2)", ctx);
    for (int k : {1, 0, -1}) {
      expect(nwd_set_decode_kernel(ctx, k), NWD_OK, "nwd_set_decode_kernel", ctx);
      expect(nwd_append_decode(ctx, q, kn, vn, kc, vc, pos, out, batch, 0, nullptr), NWD_OK,
             "nwd_append_decode(kernel choice)", ctx);
    }
    int32_t st = 0;
    auto* status = static_cast<int32_t*>(m.get(sizeof st));
    expect(nwd_append_decode_noalloc(&desc, q, kn, vn, kc, vc, pos, out, batch, 0, status, nullptr),
           NWD_OK, "nwd_append_decode_noalloc", nullptr);
    // prefill of 16 new tokens per sequence at positions 0 and 200
    const int n_new = 16;
    const int32_t pos0_h[batch] = {0, 200};
    auto* pos0 = static_cast<int32_t*>(m.get(sizeof pos0_h));
    (void)hipMemcpy(pos0, pos0_h, sizeof pos0_h, hipMemcpyHostToDevice);
    void* qp = m.get((size_t)batch * n_new * h * d * 2);
    void* op = m.get((size_t)batch * n_new * h * d * 2);
    expect(nwd_prefill_attn(ctx, qp, kc, vc, pos0, op, batch, n_new, 0, nullptr), NWD_OK,
           "nwd_prefill_attn", ctx);
    // 4-bit projections: K = 128 (4 blocks)
    const int nb = 4;
    auto* x = static_cast<float*>(m.get((size_t)batch * nb * 32 * sizeof(float)));
    Q4 w(m, 256, nb);
    auto* y = static_cast<float*>(m.get((size_t)batch * 256 * sizeof(float)));
    for (int ep : {NWD_Q4_PLAIN, NWD_Q4_RELU2, NWD_Q4_ACCUMULATE})
      expect(nwd_q4_gemv(ctx, x, &w.w, y, batch, ep, nullptr), NWD_OK, "nwd_q4_gemv", ctx);
    Q4 wq(m, h * d, nb), wk(m, hkv * d, nb), wv(m, hkv * d, nb);
    void* qo = m.get((size_t)batch * h * d * sizeof(float));
    expect(nwd_qkv_append(ctx, x, &wq.w, &wk.w, &wv.w, qo, kc, vc, pos, batch, nullptr), NWD_OK,
           "nwd_qkv_append", ctx);
    const int vocab = 1000;
    auto* logits = static_cast<float*>(m.get((size_t)batch * vocab * sizeof(float)));
    auto* ids = static_cast<uint32_t*>(m.get((size_t)batch * sizeof(uint32_t)));
    expect(nwd_argmax(ctx, logits, vocab, ids, batch, nullptr), NWD_OK, "nwd_argmax", ctx);
    Q4 wl(m, vocab, nb);
    expect(nwd_lm_head_argmax(ctx, x, &wl.w, logits, ids, batch, nullptr), NWD_OK,
           "nwd_lm_head_argmax", ctx);
    // host-side rejections on a live context
    expect(nwd_decode_attn(ctx, q, kc, vc, pos, out, batch + 1, 0, nullptr), NWD_ERR_CAPACITY,
           "nwd_decode_attn(batch > max_batch)", ctx);
    expect(nwd_prefill_attn(ctx, qp, kc, vc, pos0, op, batch, n_new, max_seq + 1, nullptr),
           NWD_ERR_CAPACITY, "nwd_prefill_attn(max_len > max_seq)", ctx);
    expect(nwd_device_status(ctx, nullptr), NWD_OK, "nwd_device_status", ctx);
    (void)hipMemcpy(&st, status, sizeof st, hipMemcpyDeviceToHost);
    if (st != 0) {
      ++g_failed;
      std::fprintf(stderr, "FAIL noalloc status %d\n", st);
    }
    if (hipDeviceSynchronize() != hipSuccess) {
      ++g_failed;
      std::fprintf(stderr, "FAIL hipDeviceSynchronize\n");
    }
  }
  nwd_destroy(ctx);
}

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
  cpu_checks();
  std::printf("nwd_abi_asan: cpu checks: %d calls, %d failed\n", g_calls, g_failed);
  std::fflush(stdout);
  if (gpu) {
    const int shapes[][2] = {{1, 128}, {2, 128}, {4, 128}, {5, 128}, {8, 128}, {3, 96}, {2, 100},
                             {7, 128}, {6, 128}, {4, 64}, {5, 256}, {12, 96}, {7, 64},
                             {7, 80}};
    for (const auto& gd : shapes) {
      const int before = g_calls;
      gpu_cycle(gd[0], gd[1]);
      std::printf("nwd_abi_asan: gpu cycle group %d head_dim %d: %d calls, %d failed so far\n",
                  gd[0], gd[1], g_calls - before, g_failed);
      std::fflush(stdout);
    }
  }
  return g_failed == 0 ? 0 : 1;
}
