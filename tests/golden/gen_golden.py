"""Generate tests/golden/fp8_golden.npz from the CPU oracle on seeded inputs.

Run from the repo root:  python tests/golden/gen_golden.py
The fixture holds small inputs and the oracle's bit-exact codes and scales (and the
fp32 GEMM values) so GPU tests can compare against committed data.  bf16 tensors are
stored as their uint16 bit patterns, fp8 codes as uint8.
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import fp8_oracle as orc  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_golden.npz")


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def main():
    g = torch.Generator().manual_seed(20240601)
    d = {}
    # activations with outliers (1% scaled by 20, as config 2), a zero row tile, a NaN and an inf tile
    x = torch.randn(128, 384, generator=g)
    x[torch.rand(128, 384, generator=g) < 0.01] *= 20
    x[5, 128:256] = 0.0
    x[7, 3] = float("nan")
    x[9, 300] = float("inf")
    x = x.to(torch.bfloat16)
    d["x_bf16"] = bf16_bits(x)
    for rs in (0, 1):
        q, s = orc.quant_rowwise(x, 128, bool(rs))
        d[f"x_row_q_rs{rs}"], d[f"x_row_s_rs{rs}"] = u8(q), s.numpy()
    # fp32 weights (master weights), tails in both dims
    w = torch.randn(200, 384, generator=g) * 0.02
    d["w_f32"] = w.numpy()
    qw, sw = orc.quant_blockwise(w, 128, 128, False)
    d["w_blk_q"], d["w_blk_s"] = u8(qw), sw.numpy()
    # GEMM fp32 values: y = x_q (x) w_q (drop the NaN/inf rows' influence by using a clean x)
    xc = torch.randn(128, 384, generator=g).to(torch.bfloat16)
    d["xc_bf16"] = bf16_bits(xc)
    qx, sx = orc.quant_rowwise(xc)
    d["xc_row_q"], d["xc_row_s"] = u8(qx), sx.numpy()
    d["y_f32"] = orc.gemm_ref(qx, sx, qw.view(torch.uint8).t().contiguous(), sw.t().contiguous()).numpy()
    # gradient tile quantization (row tiles of dy and of dy^T), round_scale on
    dy = (torch.randn(128, 200, generator=g) * 1e-3).to(torch.bfloat16)
    d["dy_bf16"] = bf16_bits(dy)
    q, s = orc.quant_rowwise(dy, 128, True)
    d["dy_row_q"], d["dy_row_s"] = u8(q), s.numpy()
    q, s = orc.quant_rowwise(dy.t().contiguous(), 128, True)
    d["dyt_row_q"], d["dyt_row_s"] = u8(q), s.numpy()
    # re-quantization of xc's row codes into 128x128 blocks (src/kernels.py:784-787)
    qb, sb = orc.quant_blockwise(orc.dequant_rowwise(qx, sx), 128, 128, False)
    d["xc_blk_q"], d["xc_blk_s"] = u8(qb), sb.numpy()
    np.savez_compressed(OUT, **d)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
