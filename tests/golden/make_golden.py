"""Write the committed golden vectors of the QIPACK linear path.

The expected outputs come from the CPU oracle (oracle/qi_oracle.c), whose
functions are pinned by the reference's known-answer tests
(int4_pack.cplus:854-938, half.cplus:81-90), closed forms and brute force in
tests/test_oracle_numerics.py.  The fixtures freeze those outputs so that a
later change to the oracle or to the kernels is caught against fixed data.

    python tests/golden/make_golden.py      # rewrites tests/golden/*.npz
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path[:0] = [str(ROOT / "oracle"), str(ROOT / "tests")]

import oracle  # noqa: E402
from _data import heavy_tailed, normal_f32, weights_f16  # noqa: E402

M, N, K = 48, 128, 512


def w4a4_case():
    x = heavy_tailed(M, K, 2024)
    x[3] = 0.0                     # all-zero row: scale 2^-24, codes 0
    x[7, :64] = 0.0
    x[7, 5] = 1000.0               # one spike in a group
    x[11] = np.where(np.arange(K) % 2 == 0, 1.0, -1.0)  # saturated +-7 after rotation
    w = weights_f16(N, K, 2025)
    a_codes, a_scales = oracle.quantize_activations(x)
    w_codes, w_scales, _ = oracle.quantize_matrix(w, 6, clip=True)
    y = oracle.w4a4_gemm(a_codes, a_scales, w_codes, w_scales)
    partials = oracle.w4a4_partials(a_codes, w_codes)
    return dict(x=x, w_f16=w, a_codes=a_codes, a_scales=a_scales, w_codes=w_codes, w_scales=w_scales, y=y,
                partials=partials.astype(np.int32))


def w4a16_case():
    x = oracle.half_from_f32(normal_f32(M, K, 2026))
    w = weights_f16(N, K, 2027)
    codes, scales, mins = oracle.quantize_matrix(w, 5)
    w_deq = oracle.w4a16_dequantize(codes, scales, mins)
    y = oracle.w4a16_gemm(x, codes, scales, mins)
    return dict(x_f16=x, w_f16=w, codes=codes, scales=scales, minimums=mins, w_dequant=w_deq, y=y)


def main():
    oracle.lib()
    np.savez_compressed(HERE / "w4a4_h256_g64.npz", **w4a4_case())
    np.savez_compressed(HERE / "w4a16_g64.npz", **w4a16_case())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
