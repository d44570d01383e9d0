// lmhead_bounds_driver.cpp -- the LM-head launch plan checked on the host,
// with no device work (tests/test_sanitizers.py builds it against the
// library's own lmhead.hip and blas_lt.cpp objects and runs it).
//
// For each shape it builds the kept-row tables, the chunking and the scratch
// sizes with the engine's functions (lmhead_rows, lmhead_shape,
// lmhead_scratch), then lmhead_check_bounds walks every thread of every
// kernel grid launch_lmhead would launch, with the kernels' own index
// functions, and the stored extent of every operand of both hipBLASLt GEMMs
// as blas_gemm describes them (gemm_layouts), against those sizes.  The first
// shape is the one whose first GPU run faulted (fp32, 32 rows with 30 kept,
// hidden 896, vocabulary 151936, tests/test_lmhead_gpu.py's targets).
// Negative controls shrink each buffer by one element and expect a report.
#include <cstdio>
#include <string>
#include <vector>

#include "../../glacier.tune_amd/csrc/lmhead_launch.hpp"

namespace {

// tests/test_lmhead_gpu.py's target pattern: dropped rows (-100 and V), the
// first and last ids, ids either side of a 4096 boundary, then spread ids.
std::vector<int32_t> targets_for(int T, int V) {
  std::vector<int32_t> t(static_cast<size_t>(T));
  const int special[] = {-100, V, 0, V - 1, 4095 < V - 1 ? 4095 : V - 1, 4096 < V - 1 ? 4096 : V - 1};
  for (int i = 0; i < T; ++i)
    t[i] = i < 6 ? special[i] : static_cast<int32_t>((static_cast<long long>(i) * 7919) % V);
  return t;
}

bool check(int T, int H, int V, bool bf16, bool grad) {
  glacier::LmHeadLaunch a{};
  a.T = T;
  a.H = H;
  a.V = V;
  a.io_bf16 = bf16;
  static char flag;
  a.d_hidden = grad ? &flag : nullptr;  // only tested against null by the plan
  const std::vector<int32_t> tg = targets_for(T, V);
  std::vector<int> rows, tgts, src_of;
  glacier::lmhead_rows(tg.data(), T, V, rows, tgts, src_of);
  glacier::lmhead_shape(a, static_cast<int>(rows.size()));
  const glacier::LmHeadScratch s = glacier::lmhead_scratch(a);
  const size_t th = static_cast<size_t>(T) * H;
  const std::string r = glacier::lmhead_check_bounds(a, s, rows.data(), tgts.data(), src_of.data(),
                                                     th, static_cast<size_t>(V) * H, grad ? th : 0);
  std::printf("T=%d H=%d V=%d %s %s: kept %d, chunk %d, ldl %d: %s\n", T, H, V,
              bf16 ? "bf16" : "fp32", grad ? "loss+grad" : "loss", a.n_valid, a.chunk, a.ldl,
              r.empty() ? "in bounds" : r.c_str());
  return r.empty();
}

// Negative controls: one element less in any one buffer must be reported.
bool detects_short_buffers(int T, int H, int V, bool bf16) {
  glacier::LmHeadLaunch a{};
  a.T = T;
  a.H = H;
  a.V = V;
  a.io_bf16 = bf16;
  static char flag;
  a.d_hidden = &flag;
  const std::vector<int32_t> tg = targets_for(T, V);
  std::vector<int> rows, tgts, src_of;
  glacier::lmhead_rows(tg.data(), T, V, rows, tgts, src_of);
  glacier::lmhead_shape(a, static_cast<int>(rows.size()));
  const glacier::LmHeadScratch full = glacier::lmhead_scratch(a);
  const size_t esz = bf16 ? 2 : 4, th = static_cast<size_t>(T) * H, vh = static_cast<size_t>(V) * H;
  bool ok = true;
  for (int which = 0; which < 8; ++which) {
    glacier::LmHeadScratch s = full;
    size_t hid = th, wt = vh, dh = th;
    switch (which) {
      case 0: s.hv -= esz; break;
      case 1: s.logits -= 4; break;
      case 2: if (!bf16) continue; s.dl -= 2; break;
      case 3: s.dhv -= 4; break;
      case 4: s.row_loss -= 4; break;
      case 5: hid -= 1; break;
      case 6: wt -= 1; break;
      case 7: dh -= 1; break;
    }
    const std::string r = glacier::lmhead_check_bounds(a, s, rows.data(), tgts.data(),
                                                       src_of.data(), hid, wt, dh);
    if (r.empty()) {
      std::printf("negative control %d (T=%d H=%d V=%d %s) was not reported\n", which, T, H, V,
                  bf16 ? "bf16" : "fp32");
      ok = false;
    }
  }
  return ok;
}

}  // namespace

int main() {
  bool ok = true;
  const int shapes[][3] = {
      {32, 896, 151936},    // the faulting case
      {37, 128, 9001},      // a padded logits row
      {512, 3584, 152064},  // Qwen2.5-7B
      {2100, 64, 262144},   // more kept rows than one 2 GB chunk holds
      {5, 8, 1},            // a one-word vocabulary
  };
  for (const auto& sh : shapes)
    for (int bf = 0; bf < 2; ++bf)
      for (int grad = 0; grad < 2; ++grad) ok = check(sh[0], sh[1], sh[2], bf != 0, grad != 0) && ok;
  for (int bf = 0; bf < 2; ++bf) {
    ok = detects_short_buffers(32, 896, 151936, bf != 0) && ok;
    ok = detects_short_buffers(2100, 64, 262144, bf != 0) && ok;
  }
  if (!ok) return 1;
  std::printf("LMHEAD_BOUNDS_OK\n");
  return 0;
}
