// Dequantizing gathers from an FP8 E5M2 cache to f32 rows: the flat, row
// and RAGGED / KV_OFFSETS kernels.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_gather_dequant_e5m2_f32(int ge, const GatherArgs &a, int64_t grid, hipStream_t s) {
  dispatch_dequant<KVX_DTYPE_F32, KVX_DTYPE_F8_E5M2>(ge, a, grid, s);
}

}  // namespace dev
}  // namespace kvx
