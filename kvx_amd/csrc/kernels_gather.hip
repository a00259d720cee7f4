// Copying gathers: gather_flat_kernel, gather_rows_kernel, the RAGGED /
// KV_OFFSETS kernels and gather_tiles_kernel over CopyOp chunks.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_gather_copy(int chunk_bytes, const GatherArgs &a, int64_t grid, hipStream_t s) {
  switch (chunk_bytes) {
    case 16: launch_gather_op<CopyOp<16>>(a, grid, s); break;
    case 8: launch_gather_op<CopyOp<8>>(a, grid, s); break;
    case 4: launch_gather_op<CopyOp<4>>(a, grid, s); break;
    case 2: launch_gather_op<CopyOp<2>>(a, grid, s); break;
    default: launch_gather_op<CopyOp<1>>(a, grid, s); break;
  }
}

void run_tiles_copy(const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid, uint32_t lds,
                    hipStream_t s) {
  launch_tiles<CopyOp<16>>(t, fmt, i64, p64, grid, lds, s);
}

}  // namespace dev
}  // namespace kvx
