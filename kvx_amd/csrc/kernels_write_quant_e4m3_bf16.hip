// Quantizing writes of bf16 rows into an FP8 E4M3 cache.
#include "kernels.h"

namespace kvx {
namespace dev {

void run_write_quant_e4m3_bf16(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s) {
  dispatch_quant<KVX_DTYPE_BF16, KVX_DTYPE_F8_E4M3>(ge, a, w, s);
}

}  // namespace dev
}  // namespace kvx
