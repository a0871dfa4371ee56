"""Write the small golden fixtures under tests/golden/.

The reference (laoyin/a100-vision-infer) commits no golden vectors for its
linear path: its tests draw random data from the CUDA RNG at run time.  These
fixtures are therefore computed here from independent library routines, not
from the CPU oracle they are used to check:

  decode_table.npy   all 256 E4M3FN codes decoded by torch.float8_e4m3fn
  block_quant.npz    a 256x384 FP32 matrix quantized per 128x128 block with the
                     recipe of tools/make_tiny_fixture.py:56-61 (amax/448 scale,
                     torch's RNE cast to float8_e4m3fn), scales row-expanded as
                     tools/fp8_import_utils.py:20 does
  linear_case.npz    y = x @ W^T for M in {1, 2, 3}: W = bf16(decode * scale) via
                     torch casts, then numpy float64 matmul, then float32 ->
                     bf16 (torch), the computation of tests/fp8_tensor_test.cpp:11-22
  swiglu_case.npz    torch.nn.functional.silu(a) * u with BF16 rounding points
                     (src/optimized.cu:73)

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def decode_table():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    return codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()


def quantize_blocks(w):
    n, k = w.shape
    nb, kb = (n + 127) // 128, (k + 127) // 128
    scales = torch.empty((nb, kb), dtype=torch.float32)
    codes = torch.empty((n, k), dtype=torch.float8_e4m3fn)
    for r in range(0, n, 128):
        for c in range(0, k, 128):
            block = w[r:r + 128, c:c + 128].float()
            scale = block.abs().max().clamp_min(1e-12) / 448
            scales[r // 128, c // 128] = scale
            codes[r:r + 128, c:c + 128] = (block / scale).to(torch.float8_e4m3fn)
    codes_u8 = codes.view(torch.uint8).numpy().copy()
    expanded = np.repeat(scales.numpy(), 128, axis=0)[:n]
    return codes_u8, scales.numpy(), np.ascontiguousarray(expanded)


def reference_linear(x_bits, codes, scales_expanded):
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32)
    k = codes.shape[1]
    s = torch.from_numpy(np.repeat(scales_expanded, 128, axis=1)[:, :k])
    w = (dec * s).to(torch.bfloat16).to(torch.float64).numpy()
    x = (x_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    y = x @ w.T
    return bf16_bits(torch.from_numpy(y.astype(np.float32)))


def main():
    np.save(os.path.join(HERE, "decode_table.npy"), decode_table())

    rng = np.random.default_rng(7)
    w = torch.from_numpy((rng.standard_normal((256, 384)) * 0.02).astype(np.float32))
    w[0:128, 256:384] = 0.0                      # an all-zero block (scale floor)
    w[130, 5] = 0.75                             # an outlier that sets its block's amax
    codes, block_scales, expanded = quantize_blocks(w)
    np.savez_compressed(os.path.join(HERE, "block_quant.npz"), w=w.numpy(), codes=codes,
                        block_scales=block_scales, scales=expanded)

    cases = {}
    for m in (1, 2, 3):
        x = bf16_bits(torch.from_numpy(rng.standard_normal((m, 384)).astype(np.float32)))
        cases[f"x{m}"] = x
        cases[f"y{m}"] = reference_linear(x, codes, expanded)
    cases["codes"] = codes
    cases["scales"] = expanded
    np.savez_compressed(os.path.join(HERE, "linear_case.npz"), **cases)

    g = torch.from_numpy(np.concatenate([
        np.linspace(-12, 12, 257, dtype=np.float32),
        (rng.standard_normal(255) * 4).astype(np.float32)])).reshape(2, 256)
    gb = g.to(torch.bfloat16)
    a, u = gb[:, :128].float(), gb[:, 128:].float()
    gate = torch.nn.functional.silu(a).to(torch.bfloat16).float()
    y = (gate * u).to(torch.bfloat16)
    np.savez_compressed(os.path.join(HERE, "swiglu_case.npz"), gate_up=bf16_bits(gb),
                        y=y.view(torch.int16).numpy().view(np.uint16))
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
