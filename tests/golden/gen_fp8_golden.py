"""Generate tests/golden/fp8_e4m3_golden.npz with torch's own casts.

Independent check of the FP8 E4M3 ("e4m3fn") conventions shared by the oracle
and the kernels (no reference counterpart: the reference has no FP8 kernels).

  quantize:   for every bf16 bit pattern x and each scale s,
              torch: (f32(x) / s).clamp(-448, 448).to(float8_e4m3fn)
              (the clamp gives saturation; torch alone maps overflow to NaN)
  dequantize: for every E4M3 code q and each scale s,
              torch: (f32(q) * s).to(bfloat16 / float16), and the f32 product
All NaN results are stored as the canonical codes the library emits (0x7F,
0x7FC0, 0x7E00, 0x7FC00000): NaN sign and payload are not part of the
contract.

Run:  python tests/golden/gen_fp8_golden.py   (CPU only, a few seconds)
"""
from pathlib import Path

import numpy as np
import torch

SCALES = np.array([1.0, 0.25, 3.0, 2.0 ** -7, 0.013671875, 1e-3, 37.5,
                   0.0044642857], dtype=np.float32)
OUT = Path(__file__).resolve().parent / "fp8_e4m3_golden.npz"


def main():
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).float()
    quant = []
    for s in SCALES.tolist():
        v = (x / torch.tensor(s, dtype=torch.float32)).clamp(-448.0, 448.0)
        q = v.to(torch.float8_e4m3fn).view(torch.uint8).clone()
        q[torch.isnan(v)] = 0x7F
        quant.append(q.numpy())
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    qf = codes.view(torch.float8_e4m3fn).float()
    deq_bf16, deq_f16, deq_f32 = [], [], []
    for s in SCALES.tolist():
        y = qf * torch.tensor(s, dtype=torch.float32)
        nan = torch.isnan(y)
        b = y.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
        h = y.to(torch.float16).view(torch.int16).numpy().view(np.uint16).copy()
        f = y.view(torch.int32).numpy().view(np.uint32).copy()
        b[nan.numpy()] = 0x7FC0
        h[nan.numpy()] = 0x7E00
        f[nan.numpy()] = 0x7FC00000
        deq_bf16.append(b)
        deq_f16.append(h)
        deq_f32.append(f)
    np.savez_compressed(OUT, scales=SCALES, quant_from_bf16=np.stack(quant),
                        dequant_bf16=np.stack(deq_bf16), dequant_f16=np.stack(deq_f16),
                        dequant_f32=np.stack(deq_f32), torch_version=np.array(torch.__version__))
    print(OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
