// Dequantizing tile gathers (gather_tiles_kernel) from an FP8 E5M2
// cache, every io dtype and table format.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_tiles_dequant_e5m2(int io, const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid,
                            uint32_t lds, hipStream_t s) {
  launch_tiles_dequant<KVX_DTYPE_F8_E5M2>(io, t, fmt, i64, p64, grid, lds, s);
}

}  // namespace dev
}  // namespace kvx
