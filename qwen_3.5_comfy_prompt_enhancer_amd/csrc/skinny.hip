// Launch routing of the skinny quantized GEMM (skinny_kernel.h): picks the K-loop
// fold structure and hands the launch to the translation unit that instantiates
// its activation / weight family.
#include <stdlib.h>
#include <string.h>

#include "qlin_internal.h"
#include "skinny_kernel.h"

namespace qlin {

// Measured: W8 decode streams best with 8-wave workgroups of short K ranges; W4
// (twice the dequantization work per byte) with 4-wave ones.
bool skinny_big(int act, int wk, int epi, int cols) {
  (void)act;
  return wk == WK_W8 && epi == EPI_STORE && cols == 8;
}

// QLIN_SKINNY_KS=any forces the run-time fold test (tuning comparisons only).
static bool force_ks_any() {
  static const bool v = [] {
    const char* e = getenv("QLIN_SKINNY_KS");
    return e && strcmp(e, "any") == 0;
  }();
  return v;
}

// The K-loop fold structure of a launch.  fp16 activations fold once per W4 group:
// statically every 4th step for group 128.  int8 activations fold per 64-wide
// activation block (and W4 sub-block of min(group, 64)): every 2nd step unless the
// W4 group is 32.
static int fold_structure(int act, int wk, int group) {
  if (act == ACT_F16) return (wk == WK_W4 && group == 128 && !force_ks_any()) ? KS_STEP4 : KS_ANY;
  if (force_ks_any() && wk == WK_W4) return KS_ANY;
  return (wk == WK_W8 || group >= 64) ? KS_STEP2 : KS_ANY;
}

hipError_t launch_skinny_pro_w8(const SkLaunch& L, const SkArgs& a, hipStream_t st);
hipError_t launch_skinny_pro_w4(const SkLaunch& L, const SkArgs& a, hipStream_t st);

// Whether a launch plan has a fused-prologue instantiation: int8 activations, the
// K-loop fold every 2nd step (W8, W4 groups of 64 or more), store or gate/up+quant
// epilogues over 64- or 128-column tiles (W8 128-column stores with up to 8 waves).
bool skinny_pro_ok(const SkLaunch& L, int group) {
  if (L.act != ACT_I8 || fold_structure(L.act, L.wk, group) != KS_STEP2) return false;
  if (L.epi != EPI_STORE && L.epi != EPI_GATEUP_Q) return false;
  if (L.cols != 4 && L.cols != 8) return false;
  if (L.hz && L.wk == WK_W8) return false;
  const int maxw = (L.cols == 4) ? 8 : ((L.wk == WK_W8 && L.epi == EPI_STORE) ? 8 : 4);
  return L.waves <= maxw;
}

hipError_t launch_skinny(const SkLaunch& L0, const SkArgs& a, hipStream_t st) {
  SkLaunch L = L0;
  L.ks = fold_structure(L.act, L.wk, a.group);
  if (L.pro) {
    if (!skinny_pro_ok(L, a.group)) return hipErrorInvalidValue;
    return (L.wk == WK_W8) ? launch_skinny_pro_w8(L, a, st) : launch_skinny_pro_w4(L, a, st);
  }
  if (L.act == ACT_F16) return launch_skinny_f16(L, a, st);
  return (L.wk == WK_W8) ? launch_skinny_i8w8(L, a, st) : launch_skinny_i8w4(L, a, st);
}

}  // namespace qlin
