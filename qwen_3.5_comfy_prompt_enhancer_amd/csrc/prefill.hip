// Prefill GEMM for fp16 activations with more than 16 rows (the kernel is in
// prefill_kernel.h): the W8 instantiations, the plan geometry and the dispatch by
// weight kind and W4 scale dtype.
#include "prefill_kernel.h"

namespace qlin {

void prefill_geometry(int shape, int* bm, int* bn, int* waves) {
  using G0 = Geo<WK_W8, 1, 2, 1>;
  using G1 = Geo<WK_W8, 2, 4, 1>;
  using G2 = Geo<WK_W8, 1, 2, 2>;
  if (shape == PF_128x128) *bm = G0::BM, *bn = G0::BN, *waves = G0::WAVES;
  else if (shape == PF_128x128_K2) *bm = G2::BM, *bn = G2::BN, *waves = G2::WAVES;
  else *bm = G1::BM, *bn = G1::BN, *waves = G1::WAVES;
}

bool prefill_shape_ok(int shape) { return shape >= 0 && shape < PF_SHAPES; }

bool prefill_balanced_ok(long long tiles, int nkt, int sk) {
  if (sk < 2 || nkt < 1) return false;
  for (long long t = 0; t < tiles; ++t) {
    const long long u0 = t * nkt, u1 = u0 + nkt - 1;
    if (u1 / sk - u0 / sk > 1) return false;  // three or more workgroups on the tile
  }
  return true;
}

hipError_t launch_prefill(const TlArgs& a, int wk, bool hz, int shape, hipStream_t st) {
  if (wk == WK_W8) return launch_prefill_kind<WK_W8, false, 0>(a, shape, st);
  switch (a.sdt) {
    case DT_F16: return launch_prefill_w4_f16(a, hz, shape, st);
    case DT_BF16: return launch_prefill_w4_bf16(a, hz, shape, st);
    case DT_F32: return launch_prefill_w4_f32(a, hz, shape, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qlin

