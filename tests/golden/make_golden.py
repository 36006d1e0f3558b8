"""Write the golden fixtures under tests/golden/ by running apus's OWN CPU kernels
(compiled from the apus sources into oracle/_ref/libapus_ref.so; needs the
apus checkout, so it runs where the sources are, never on the GPU box).

The reference keeps no committed fixtures: its generators (tests/m3/gen_golden.py,
tests/m4a/gen_golden.py) are regenerated on demand. These fixtures follow
their shapes and corner cases (m3: M=3, O=64, K=256 with zero / +-6 / clamp
blocks; m4a: M=8, O=320, K=384 with zero tiles, +-448, min-subnormal codes,
scale bytes 0/1/200/254), with the expected outputs produced by the compiled
reference itself:
  act.npz : x -> BF16 round + per-128 act quant (apus_act_quant_rows, c/attn.h:393)
  fp4.npz : apus_fp4_gemm_scalar (c/fp4.h:367) and apus_fp4_linear (c/attn.h:432)
  fp8.npz : apus_fp8_gemm_scalar (c/fp8.h:191) and apus_fp8_linear (c/attn.h:408)
  moe.npz : routed output of apus_moe_forward (c/moe.h:369, ApusMoeInterm.moe_routed)
Run:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

from pyoracle import Reference, bf16_round_np  # noqa: E402


def act_case(rng):
    x = (rng.standard_normal((7, 384)) * 3.0).astype(np.float32)
    x[1] = 0.0                              # amax floor
    x[2, :128] *= 1e4                       # outliers
    x[3] = 1e-30                            # tiny
    x[4] = -np.abs(x[4])                    # all negative
    x[5, ::5] = 3584.0                      # exact power-of-two amax
    x[6, 200] = 1e38                        # huge finite
    return x


def fp4_case(rng):
    M, O, K = 3, 64, 256
    w = rng.integers(0, 256, (O, K // 2), dtype=np.uint8)
    ws = rng.integers(118, 131, (O, K // 32), dtype=np.uint8)
    w[0, 0:16] = 0x00; ws[0, 0] = 200      # zero block under a huge scale
    w[1, 16:32] = 0x77                      # +6 everywhere
    w[2, 32:48] = 0xFF                      # -6 everywhere
    w[3, 48:64] = 0x10                      # 0 / 0.5
    ws[4, 4] = 0; ws[5, 5] = 1              # subnormal / tiny scales
    w[6, 96:112] = 0x00; ws[6, 6] = 254     # 2^127 on a zero block
    x = (rng.standard_normal((M, K)) * 3.0).astype(np.float32)
    x[1] = 0.0                              # zero row
    x[2, 128:] *= 100.0                     # large second group
    return w, ws, x


def fp8_case(rng):
    M, O, K = 8, 320, 384
    from helpers import e4m3_np
    w = e4m3_np(np.clip(rng.standard_normal((O, K)), -448, 448).astype(np.float32))
    ws = rng.integers(117, 124, ((O + 127) // 128, K // 128), dtype=np.uint8)
    w[0:128, 0:128] = 0; ws[0, 0] = 254     # zero tile under a huge scale
    w[130, :64] = 0x7E; w[131, :64] = 0xFE  # +-448
    w[132, :] = 0x01                        # min subnormal
    ws[1, 1] = 0; ws[2, 2] = 1; ws[1, 2] = 200
    x = (rng.standard_normal((M, K)) * 2.0).astype(np.float32)
    x[3] = 0.0
    return w, ws, x


def moe_case(rng):
    E, dim, inter, s, topk = 4, 256, 128, 4, 2
    experts = []
    for _ in range(E):
        experts.append((rng.integers(0, 256, (inter, dim // 2), dtype=np.uint8),
                        rng.integers(118, 131, (inter, dim // 32), dtype=np.uint8),
                        rng.integers(0, 256, (dim, inter // 2), dtype=np.uint8),
                        rng.integers(118, 131, (dim, inter // 32), dtype=np.uint8),
                        rng.integers(0, 256, (inter, dim // 2), dtype=np.uint8),
                        rng.integers(118, 131, (inter, dim // 32), dtype=np.uint8)))
    gate = (rng.standard_normal((E, dim)) * 0.05).astype(np.float32)
    x = bf16_round_np(rng.standard_normal((s, dim)).astype(np.float32))
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(s)]).astype(np.int32)
    return experts, gate, x, idx


def main():
    R = Reference()
    rng = np.random.default_rng(20260729)
    out = {}

    x = act_case(rng)
    codes, sc = R.act_quant(x)
    out["act.npz"] = dict(x=x, codes=codes, scales=sc)

    w, ws, x = fp4_case(rng)
    c, s = R.act_quant(x)
    out["fp4.npz"] = dict(w=w, ws=ws, x=x, codes=c, scales=s,
                          gemm=R.fp4_gemm_scalar(w, ws, c, s), linear=R.fp4_linear(w, ws, x))

    w, ws, x = fp8_case(rng)
    c, s = R.act_quant(x)
    out["fp8.npz"] = dict(w=w, ws=ws, x=x, codes=c, scales=s,
                          gemm=R.fp8_gemm_scalar(w, ws, c, s), linear=R.fp8_linear(w, ws, x))

    experts, gate, x, idx = moe_case(rng)
    rw, ry = R.moe_routed(experts, gate, x, idx, 1.5, 10.0)
    d = dict(x=x, idx=idx, wgt=rw, y=ry, limit=np.float32(10.0))
    for e, tensors in enumerate(experts):
        for name, t in zip(("w1", "w1s", "w2", "w2s", "w3", "w3s"), tensors):
            d[f"e{e}_{name}"] = t
    out["moe.npz"] = d

    lines = []
    for name, arrays in out.items():
        path = os.path.join(HERE, name)
        np.savez(path, **arrays)
        lines.append(f"{hashlib.sha256(open(path, 'rb').read()).hexdigest()}  {name}")
    with open(os.path.join(HERE, "SHA256SUMS"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


if __name__ == "__main__":
    main()
