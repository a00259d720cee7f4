// Copying writes: write_flat_kernel, write_kernel and write_tiles_kernel
// over CopyOp chunks.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_write_copy(int chunk_bytes, const WriteArgs &a, const WriteLaunch &w, hipStream_t s) {
  switch (chunk_bytes) {
    case 16: launch_write_op<CopyOp<16>>(a, w, s); break;
    case 8: launch_write_op<CopyOp<8>>(a, w, s); break;
    case 4: launch_write_op<CopyOp<4>>(a, w, s); break;
    case 2: launch_write_op<CopyOp<2>>(a, w, s); break;
    default: launch_write_op<CopyOp<1>>(a, w, s); break;
  }
}

}  // namespace dev
}  // namespace kvx
