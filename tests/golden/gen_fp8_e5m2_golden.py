"""Generate tests/golden/fp8_e5m2_golden.npz with torch's own casts.

Independent check of the FP8 E5M2 conventions shared by the oracle and the
kernels (no reference counterpart: the reference has no FP8 kernels).

  quantize:   for every bf16 and every f16 bit pattern x and each scale s,
              torch: (f32(x) / s).clamp(-57344, 57344).to(float8_e5m2)
              (the clamp gives saturation, infinities included; torch alone
              rounds overflow to infinity)
  dequantize: for every E5M2 code q and each scale s,
              torch: (f32(q) * s).to(bfloat16 / float16), and the f32 product
All NaN results are stored as the canonical codes the library emits (0x7E,
0x7FC0, 0x7E00, 0x7FC00000): NaN sign and payload are not part of the
contract.

Run:  python tests/golden/gen_fp8_e5m2_golden.py   (CPU only, a few seconds)
"""
from pathlib import Path

import numpy as np
import torch

SCALES = np.array([1.0, 0.25, 3.0, 2.0 ** -7, 0.013671875, 1e-3, 37.5,
                   0.0044642857], dtype=np.float32)
OUT = Path(__file__).resolve().parent / "fp8_e5m2_golden.npz"
MAX = 57344.0


def quant(x: torch.Tensor, s: float) -> np.ndarray:
    v = (x / torch.tensor(s, dtype=torch.float32)).clamp(-MAX, MAX)
    q = v.to(torch.float8_e5m2).view(torch.uint8).clone()
    q[torch.isnan(v)] = 0x7E
    return q.numpy()


def main():
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    xb = bits.view(torch.bfloat16).float()
    xh = bits.view(torch.float16).float()
    quant_bf16 = [quant(xb, s) for s in SCALES.tolist()]
    quant_f16 = [quant(xh, s) for s in SCALES.tolist()]
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    qf = codes.view(torch.float8_e5m2).float()
    deq_bf16, deq_f16, deq_f32 = [], [], []
    for s in SCALES.tolist():
        y = qf * torch.tensor(s, dtype=torch.float32)
        nan = torch.isnan(y).numpy()
        b = y.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
        h = y.to(torch.float16).view(torch.int16).numpy().view(np.uint16).copy()
        f = y.view(torch.int32).numpy().view(np.uint32).copy()
        b[nan] = 0x7FC0
        h[nan] = 0x7E00
        f[nan] = 0x7FC00000
        deq_bf16.append(b)
        deq_f16.append(h)
        deq_f32.append(f)
    np.savez_compressed(OUT, scales=SCALES, quant_from_bf16=np.stack(quant_bf16),
                        quant_from_f16=np.stack(quant_f16),
                        dequant_bf16=np.stack(deq_bf16), dequant_f16=np.stack(deq_f16),
                        dequant_f32=np.stack(deq_f32), torch_version=np.array(torch.__version__))
    print(OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
