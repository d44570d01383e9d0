// abi_asan_driver.cpp -- the C ABI's host-side checks under AddressSanitizer
// and UndefinedBehaviorSanitizer, on a machine without a GPU
// (tests/test_sanitizers.py builds every library source host-only with the
// sanitizers on the host pass, links this driver, and runs it).
//
// Every call here must be refused before any device work: argument checks
// (null pointers, bad descriptors, cu_seqlens arrays that are not offsets,
// head counts, dtypes, sizes), context creation without a device, and the
// small queries.  Arrays are exactly-sized heap blocks, so a check that reads
// past what the caller passed aborts the run.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/glacier_attn.h"
#include "../../include/glacier_lmhead.h"
#include "../../include/glacier_lora_file.h"
#include "../../include/glacier_norm.h"
#include "../../include/glacier_qkv.h"

namespace {

int g_fail = 0;

void expect(int rc, int want, const char* what) {
  const char* msg = glacier_attn_last_error();
  if (rc != want) {
    std::fprintf(stderr, "%s: status %d, expected %d (%s)\n", what, rc, want, msg);
    g_fail = 1;
  } else if (rc != GLACIER_ATTN_OK && (msg == nullptr || msg[0] == '\0')) {
    std::fprintf(stderr, "%s: status %d without an error text\n", what, rc);
    g_fail = 1;
  }
}

// cu_seqlens as its own exactly-sized heap block
struct Cu {
  int32_t* p;
  explicit Cu(std::vector<int32_t> v) : p(static_cast<int32_t*>(std::malloc(v.size() * 4))) {
    std::memcpy(p, v.data(), v.size() * 4);
  }
  ~Cu() { std::free(p); }
};

glacier_attn_desc desc(int T, int n_seqs, const int32_t* cu, int hq, int hkv, int d,
                       int prec = GLACIER_ATTN_PREC_BF16, int io = GLACIER_ATTN_IO_BF16,
                       float base = 1.0e4f) {
  glacier_attn_desc x;
  x.total_tokens = T;
  x.n_seqs = n_seqs;
  x.cu_seqlens = cu;
  x.n_heads_q = hq;
  x.n_heads_kv = hkv;
  x.head_dim = d;
  x.rope_freq_base = base;
  x.precision = prec;
  x.io_dtype = io;
  return x;
}

typedef int (*AttnFn)(const glacier_attn_desc*);

int call_forward(const glacier_attn_desc* d) {
  return glacier_attn_forward(nullptr, d, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                              nullptr);
}
int call_backward(const glacier_attn_desc* d) {
  return glacier_attn_backward(nullptr, d, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                               nullptr, nullptr, nullptr);
}
int call_noalloc(const glacier_attn_desc* d) {
  return glacier_attn_backward_noalloc(nullptr, d, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, nullptr, nullptr, nullptr);
}

void attention_descriptors() {
  const AttnFn fns[] = {call_forward, call_backward, call_noalloc};
  for (AttnFn fn : fns) {
    expect(fn(nullptr), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "NULL desc");
    Cu dec({0, 5, 3, 9});
    glacier_attn_desc x = desc(9, 3, dec.p, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "decreasing cu_seqlens");
    Cu first({2, 5, 9});
    x = desc(9, 2, first.p, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens[0] != 0");
    Cu last({0, 4, 9});
    x = desc(10, 2, last.p, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens[n] != T");
    x = desc(9, 3, nullptr, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "n_seqs > 1 without cu_seqlens");
    x = desc(9, 0, nullptr, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "n_seqs = 0");
    x = desc(-1, 1, nullptr, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "negative T");
    x = desc(9, 1, nullptr, 3, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "Hq % Hkv");
    x = desc(9, 1, nullptr, 4, 0, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "Hkv = 0");
    x = desc(9, 1, nullptr, 4, 2, 2000);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "head_dim > 1024");
    x = desc(9, 1, nullptr, 4, 2, 300);
    expect(fn(&x), GLACIER_ATTN_ERR_UNSUPPORTED, "head_dim 300");
    // 80 runs on padded rows (only the context is missing), except in the
    // allocation-free backward, which takes the built sizes only
    x = desc(9, 1, nullptr, 4, 2, 80);
    expect(fn(&x), fn == call_noalloc ? GLACIER_ATTN_ERR_UNSUPPORTED : GLACIER_ATTN_ERR_INVALID_ARGUMENT,
           "head_dim 80");
    x = desc(9, 1, nullptr, 4, 2, 200, GLACIER_ATTN_PREC_FP32, GLACIER_ATTN_IO_F32);
    expect(fn(&x), GLACIER_ATTN_ERR_UNSUPPORTED, "head_dim 200 (padded to 256) in the fp32 mode");
    x = desc(9, 1, nullptr, 4, 2, 256, GLACIER_ATTN_PREC_FP32, GLACIER_ATTN_IO_F32);
    expect(fn(&x), GLACIER_ATTN_ERR_UNSUPPORTED, "head_dim 256 in the fp32 mode");
    x = desc(9, 1, nullptr, 4, 2, 64, 7);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "precision");
    x = desc(9, 1, nullptr, 4, 2, 64, GLACIER_ATTN_PREC_FP32, GLACIER_ATTN_IO_BF16);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "bf16 tensors in fp32 mode");
    x = desc(9, 1, nullptr, 4, 2, 64, GLACIER_ATTN_PREC_BF16, GLACIER_ATTN_IO_BF16, -1.0f);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "theta <= 0");
    x = desc(70000, 1, nullptr, 4, 2, 64);
    expect(fn(&x), GLACIER_ATTN_ERR_UNSUPPORTED, "sequence too long");
    // a long valid packing: every offset is read, then only the context is missing
    std::vector<int32_t> many(1025);
    for (int b = 0; b <= 1024; ++b) many[b] = 3 * b;
    Cu big(many);
    x = desc(3 * 1024, 1024, big.p, 4, 2, 128);
    expect(fn(&x), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "missing context");
  }
}

void host_entry_points() {
  std::vector<float> q(8 * 3 * 64), k(8 * 2 * 64), out(8 * 3 * 64);
  expect(glacier_attn_forward_host(nullptr, 0, q.data(), k.data(), k.data(), out.data(), nullptr, 8,
                                   3, 2, 64, 1e4f),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "forward_host Hq % Hkv");
  expect(glacier_attn_forward_host(nullptr, 0, q.data(), k.data(), k.data(), out.data(), nullptr, 8,
                                   2, 2, 300, 1e4f),
         GLACIER_ATTN_ERR_UNSUPPORTED, "forward_host head_dim 300");
  expect(glacier_attn_forward_host(nullptr, 0, q.data(), k.data(), k.data(), out.data(), nullptr, 8,
                                   2, 2, 64, 1e4f),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "forward_host without a context");
  expect(glacier_attn_backward_host(nullptr, 0, q.data(), q.data(), k.data(), k.data(), q.data(),
                                    nullptr, q.data(), k.data(), k.data(), 8, 2, 2, 64, 1e4f),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "backward_host without lse");
}

void projections() {
  glacier_proj_desc d{4, 16, 2, GLACIER_ATTN_PREC_FP32, GLACIER_ATTN_IO_F32};
  std::vector<float> x(4 * 16), w(8 * 16), y(4 * 8), a(16 * 2);
  glacier_lora_proj p{};
  p.w = w.data();
  p.out_features = 8;
  p.y = y.data();
  p.lora_a = a.data();  // without lora_b
  p.scaling = 1.0f;
  expect(glacier_proj_forward(nullptr, nullptr, x.data(), &p, 1), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "proj NULL desc");
  expect(glacier_proj_forward(nullptr, &d, x.data(), &p, 1), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "proj lora_a without lora_b");
  expect(glacier_proj_forward(nullptr, &d, x.data(), &p, 0), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "proj n_proj 0");
  expect(glacier_proj_forward(nullptr, &d, x.data(), &p, GLACIER_PROJ_MAX_PROJ + 1),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "proj n_proj too large");
  glacier_proj_desc bad = d;
  bad.in_features = 0;
  expect(glacier_proj_forward(nullptr, &bad, x.data(), &p, 1), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "proj in_features 0");
  bad = d;
  bad.io_dtype = GLACIER_ATTN_IO_BF16;
  expect(glacier_proj_backward(nullptr, &bad, x.data(), &p, 1, nullptr),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "proj bf16 tensors in fp32 mode");
}

void norms_and_lmhead() {
  std::vector<float> x(4 * 8), w(8), y(4 * 8);
  glacier_norm_desc nd{4, 8, GLACIER_ATTN_IO_F32, 1e-6f};
  expect(glacier_rmsnorm_forward(nullptr, nullptr, x.data(), nullptr, w.data(), nullptr, y.data()),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "norm NULL desc");
  glacier_norm_desc bad = nd;
  bad.n = 6;
  expect(glacier_rmsnorm_forward(nullptr, &bad, x.data(), nullptr, w.data(), nullptr, y.data()),
         GLACIER_ATTN_ERR_UNSUPPORTED, "norm n % 4");
  bad = nd;
  bad.eps = -1.0f;
  expect(glacier_rmsnorm_backward(nullptr, &bad, y.data(), x.data(), w.data(), nullptr, x.data(),
                                  nullptr),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "norm eps < 0");
  expect(glacier_rmsnorm_forward(nullptr, &nd, x.data(), nullptr, w.data(), nullptr, y.data()),
         GLACIER_ATTN_ERR_INVALID_ARGUMENT, "norm without a context");
  glacier_lmhead_desc ld{4, 8, 16, GLACIER_ATTN_PREC_FP32, GLACIER_ATTN_IO_F32};
  std::vector<int32_t> t(4, 1);
  float loss = 0.0f;
  int32_t nv = 0;
  const int rc = glacier_lmhead_loss(nullptr, &ld, x.data(), t.data(), w.data(), &loss, &nv);
  if (rc == GLACIER_ATTN_OK) {
    std::fprintf(stderr, "lmhead without a context succeeded\n");
    g_fail = 1;
  }
}

void queries_and_context() {
  if (glacier_attn_supports(512, 128) != 1 || glacier_attn_supports(512, 80) != 1 ||
      glacier_attn_supports(512, 300) != 0 || glacier_attn_supports(0, 64) != 0) {
    std::fprintf(stderr, "glacier_attn_supports gate\n");
    g_fail = 1;
  }
  const int n = glacier_attn_kernel_count();
  for (int i = -1; i <= n; ++i) (void)glacier_attn_kernel_name(i);
  glacier_attn_ctx* ctx = nullptr;
  const int rc = glacier_attn_create(0, GLACIER_ATTN_PREC_BF16, &ctx);
  if (rc == GLACIER_ATTN_OK) {
    // a device is present after all: nothing more to check on the host
    glacier_attn_destroy(ctx);
  } else if (ctx != nullptr) {
    std::fprintf(stderr, "failed create left a context\n");
    g_fail = 1;
  }
  expect(glacier_attn_create(0, 9, &ctx), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "create precision");
  expect(glacier_attn_create(0, GLACIER_ATTN_PREC_BF16, nullptr), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "create NULL out");
  expect(glacier_attn_synchronize(nullptr), GLACIER_ATTN_ERR_INVALID_ARGUMENT, "synchronize NULL");
  expect(glacier_attn_set_stream(nullptr, nullptr), GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "set_stream NULL");
  glacier_attn_destroy(nullptr);
}

}  // namespace

int main() {
  attention_descriptors();
  host_entry_points();
  projections();
  norms_and_lmhead();
  queries_and_context();
  if (g_fail) return 1;
  std::printf("ABI_SANITIZE_OK\n");
  return 0;
}
