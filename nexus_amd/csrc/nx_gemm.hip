// nx_gemm.hip — prefill path: grouped GEMM on MFMA (placeholder until the
// LDS-dequant kernels land; the launchers report the path as unsupported).
#include "nx_internal.hpp"

namespace nx {
int gemm_tile_m() { return 128; }
int launch_gemm_gateup(nx_ctx *, const GemmPlan &) { return fail(NX_ERR_UNSUPPORTED, "MFMA path not built"); }
int launch_gemm_down(nx_ctx *, const GemmPlan &) { return fail(NX_ERR_UNSUPPORTED, "MFMA path not built"); }
}  // namespace nx
