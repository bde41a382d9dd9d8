"""Write the codec golden vectors used by tests/test_oracle_codecs.py.

The expected outputs come from torch's own bfloat16 / float8_e4m3fn /
float8_e5m2 conversion routines (an independent library implementation of
the same IEEE / OCP round-to-nearest-even casts), not from the oracle. Run:

    python tests/golden/make_golden.py

which rewrites tests/golden/codec_vectors.npz (about 100 KB).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "codec_vectors.npz"


def structured_inputs() -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(20261201))
    pieces = []
    # boundaries of the fp8 formats and their ties, with neighbours
    anchors = [0.0, 2.0 ** -10, 2.0 ** -9, 2.0 ** -7, 2.0 ** -6, 2.0 ** -17, 2.0 ** -16,
               2.0 ** -15, 2.0 ** -14, 0.5, 1.0, 1.0625, 1.125, 1.1875, 240.0, 256.0, 416.0,
               432.0, 448.0, 456.0, 464.0, 465.0, 480.0, 49152.0, 57344.0, 61440.0, 65536.0]
    for a in anchors:
        bits = np.float32(a).view(np.uint32).astype(np.int64)
        for d in range(-4, 5):
            pieces.append(np.uint32(max(bits + d, 0)))
    base = np.array(pieces, dtype=np.uint32)
    rand = rng.integers(0, 2 ** 32, size=6000, dtype=np.uint64).astype(np.uint32)
    small = (rng.standard_normal(4000) * rng.choice([1e-3, 1.0, 30.0, 500.0], size=4000))
    specials = np.array([np.inf, -np.inf, np.nan, -0.0, 1e-45, -1e-45], np.float32)
    x = np.concatenate([base.view(np.float32), -base.view(np.float32), rand.view(np.float32),
                        small.astype(np.float32), specials])
    return x.astype(np.float32)


def main() -> None:
    x = structured_inputs()
    t = torch.from_numpy(x.copy())
    bf16 = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    e4m3 = t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    e5m2 = t.to(torch.float8_e5m2).view(torch.uint8).numpy()
    codes = torch.arange(256, dtype=torch.uint8)
    dec_e4m3 = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    dec_e5m2 = codes.view(torch.float8_e5m2).to(torch.float32).numpy()
    np.savez_compressed(OUT, x=x, bf16=bf16, e4m3fn=e4m3, e5m2=e5m2, dec_e4m3fn=dec_e4m3,
                        dec_e5m2=dec_e5m2, torch_version=np.array(torch.__version__))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {x.size} inputs)")


if __name__ == "__main__":
    main()
