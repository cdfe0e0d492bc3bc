"""Write tests/golden/triton_floor.npz: what Triton's own typing rules give for the tile
amax floor of src/kernels.py:51-53 (row-wise) and :112-114 (block-wise) on zero and tiny
bf16 / fp16 / fp32 tiles.

FIXTURE GENERATION ONLY, run in the build container (it needs the installed Triton and
runs its CPU interpreter); no test, GPU run or product code imports it.  The committed
fixture is data: inputs (as bit patterns) and the interpreter's scales and codes.

    TRITON_INTERPRET=1 python tests/golden/gen_triton_floor.py

The two kernels below are this build's own minimal restatement of the quantizer
arithmetic, written in Triton only so that Triton decides the operand types:
    a = tl.maximum(tl.max(tl.abs(x)), 1e-4);  s = a / 448  (or exp2(ceil(log2(a / 448))))
    y = clamp(x / s, -448, 448)
tl.max widens bf16/fp16 to fp32 before it reduces, so the floor is fp32(1e-4) for every
input dtype.  The kernels store the scale and the fp32 value y; the codes in the fixture
are y cast by torch's CPU cast (pinned to a textbook e4m3fn round-to-nearest-even by
tests/test_oracle.py).  The interpreter's own .to(tl.float8e4nv) is a numpy emulation
that does not carry a rounding into the next binade (0.4978 -> 0.25), so it is not used.
tests/test_oracle.py compares the oracle's quantizers with these scales and codes.
The interpreter is Triton 3.6.0 (the reference pins 3.5.1, uv.lock:2385-2386).
"""
import os

os.environ.setdefault("TRITON_INTERPRET", "1")

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "triton_floor.npz")


@triton.jit
def _row_tiles(x_ptr, y_ptr, s_ptr, N, nb, ROUND: tl.constexpr, BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cb = tl.program_id(1)
    cols = cb * BLOCK + tl.arange(0, BLOCK)
    m = cols < N
    x = tl.load(x_ptr + row * N + cols, mask=m, other=0.0)
    a = tl.maximum(tl.max(tl.abs(x)), 1e-4)
    if ROUND:
        s = tl.exp2(tl.ceil(tl.log2(a / 448.0)))
    else:
        s = a / 448.0
    y = tl.minimum(tl.maximum(x / s, -448.0), 448.0)
    tl.store(y_ptr + row * N + cols, y, mask=m)
    tl.store(s_ptr + row * nb + cb, s)


@triton.jit
def _block_tiles(x_ptr, y_ptr, s_ptr, M, N, nb, BLOCK: tl.constexpr):
    rb = tl.program_id(0)
    cb = tl.program_id(1)
    rows = rb * BLOCK + tl.arange(0, BLOCK)
    cols = cb * BLOCK + tl.arange(0, BLOCK)
    m = (rows[:, None] < M) & (cols[None, :] < N)
    off = rows[:, None] * N + cols[None, :]
    x = tl.load(x_ptr + off, mask=m, other=0.0)
    a = tl.maximum(tl.max(tl.abs(x)), 1e-4)
    s = a / 448.0
    y = tl.minimum(tl.maximum(x / s, -448.0), 448.0)
    tl.store(y_ptr + off, y, mask=m)
    tl.store(s_ptr + rb * nb + cb, s)


def _bits(t):
    t = t.contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def _row_input(dt, g):
    """[16, 200]: row tiles that are zero, -0, gradient-sized, at the floor's edges, with a
    NaN among tiny values, and ordinary; the second tile of each row is a 72-wide tail."""
    x = torch.randn(16, 200, generator=g) * 2e-5
    x[0] = 0.0
    x[1] = -0.0
    x[2, :128] = torch.randn(128, generator=g) * 1e-7      # deep below the floor
    x[3, 5] = float("nan")
    x[4] = torch.randn(200, generator=g)                  # ordinary tiles
    x[5, 130:] = 0.0                                      # zero tail tile
    x = x.to(dt)
    # amax exactly on, just below and just above fp32(1e-4) as far as the dtype allows
    f32_floor = torch.tensor(1e-4, dtype=torch.float32)
    below = torch.nextafter(f32_floor.to(dt).float(), torch.tensor(0.0)).to(dt)
    for r, v in ((6, f32_floor.to(dt)), (7, below), (8, torch.tensor(1e-4).to(dt))):
        x[r, 17] = v
        x[r, 150] = -v
    # the largest value of a 16-bit dtype below fp32(1e-4), and the smallest at or above it
    if dt != torch.float32:
        every = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(dt).float()
        x[9, 0] = every[(every < f32_floor) & (every > 0)].max().to(dt)
        x[10, 0] = every[every >= f32_floor].min().to(dt)
    return x


def _block_input(dt, g):
    """[128, 264]: block 0 gradient-sized with a NaN, block 1 zero, block 2 an 8-wide
    ordinary tail."""
    x = torch.randn(128, 264, generator=g) * 2e-5
    x[70, 33] = float("nan")
    x[:, 128:256] = 0.0
    x[:, 256:] = torch.randn(128, 8, generator=g)
    return x.to(dt)


def _codes(y):
    return y.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def main():
    g = torch.Generator().manual_seed(77)
    d = {}
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)):
        x = _row_input(dt, g)
        M, N = x.shape
        nb = (N + 127) // 128
        d[f"row_x_{name}"] = _bits(x)
        for rs in (0, 1):
            y = torch.zeros(M, N, dtype=torch.float32)
            s = torch.zeros(M, nb, dtype=torch.float32)
            _row_tiles[(M, nb)](x, y, s, N, nb, ROUND=rs, BLOCK=128)
            d[f"row_q_{name}_rs{rs}"] = _codes(y)
            d[f"row_s_{name}_rs{rs}"] = s.numpy()
        xb = _block_input(dt, g)
        M, N = xb.shape
        nbn = (N + 127) // 128
        y = torch.zeros(M, N, dtype=torch.float32)
        s = torch.zeros((M + 127) // 128, nbn, dtype=torch.float32)
        _block_tiles[((M + 127) // 128, nbn)](xb, y, s, M, N, nbn, BLOCK=128)
        d[f"blk_x_{name}"] = _bits(xb)
        d[f"blk_q_{name}"] = _codes(y)
        d[f"blk_s_{name}"] = s.numpy()
    d["triton_version"] = np.array(triton.__version__)
    np.savez_compressed(OUT, **d)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
