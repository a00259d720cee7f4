// Dequantizing gathers from an FP8 E5M2 cache to bf16 rows: the flat, row
// and RAGGED / KV_OFFSETS kernels.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_gather_dequant_e5m2_bf16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s) {
  dispatch_dequant<KVX_DTYPE_BF16, KVX_DTYPE_F8_E5M2>(ge, a, grid, s);
}

}  // namespace dev
}  // namespace kvx
