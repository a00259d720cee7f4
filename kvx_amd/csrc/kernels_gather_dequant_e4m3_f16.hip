// Dequantizing gathers from an FP8 E4M3 cache to f16 rows: the flat, row
// and RAGGED / KV_OFFSETS kernels.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_gather_dequant_e4m3_f16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s) {
  dispatch_dequant<KVX_DTYPE_F16, KVX_DTYPE_F8_E4M3>(ge, a, grid, s);
}

}  // namespace dev
}  // namespace kvx
