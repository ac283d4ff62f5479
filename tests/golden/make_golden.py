"""Write the golden fixtures in this folder from the reference implementation itself.

Runs only where the reference checkout is present (its path is the first argument,
default /root/reference); the fixtures it writes are committed, and the tests read
them without the reference. What is imported and why:

* wisp/quant.py (pure torch): `quantize` and `dequant` on seeded inputs. Our oracle
  restates them from IEEE closed forms; these fixtures check that the restatement
  matches torch's own CPU kernels bit for bit (division, round-half-even, fp16 and
  bf16 casts) on real data, which no closed form or invariant can confirm.
* wisp/kernels.py under TRITON_INTERPRET=1 (Triton's CPU interpreter, as the
  reference's tests/test_kernels.py:3 runs it): the reference kernels' own outputs
  for moe_decode_q4, moe_decode_q4_fast, moe_decode_q3_fast and rope_decode, so the
  HIP kernels are compared with what the reference computes, not only with our
  fp64 restatement.

Inputs are regenerated from numpy's legacy RandomState (a frozen stream), so the
fixture stores seeds plus the sha256 of every input and output, and the small
outputs in full. Output: golden.json beside this script.

The interpreter stores float32 into bf16 pointers by truncation, so the bf16
outputs of the Triton kernels that store them (moe_decode_q4_fast,
moe_decode_q3_fast, rope_decode in bf16) are the truncated float32 results;
moe_decode_q4's final sum and cast are torch ops and round to nearest even.

Usage:  python tests/golden/make_golden.py [/root/reference]
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "golden.json")

# shapes: the reference's own kernel-test shape (test_kernels.py:23, H=256 I=128 G=128)
H, I, G = 256, 128, 128
N = H * I
N_EXPERTS = 4


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def expert_input(seed: int) -> np.ndarray:
    """bf16 bits [3, n] of 0.05 * N(0,1): float32 rounded to bf16 by torch (RTNE)."""
    import torch

    w = (np.random.RandomState(seed).standard_normal((3, N)) * 0.05).astype(np.float32)
    return torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def x_input(seed: int) -> np.ndarray:
    import torch

    x = np.random.RandomState(seed).standard_normal(H).astype(np.float32)
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main(ref_root: str) -> None:
    os.environ["TRITON_INTERPRET"] = "1"
    sys.dont_write_bytecode = True  # the reference checkout is read-only: no __pycache__ there
    sys.path.insert(0, ref_root)
    import torch
    from wisp import kernels as RK  # noqa: E402  (the reference, this container only)
    from wisp import quant as RQ  # noqa: E402

    def bf16(bits: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)

    def bits16(t: torch.Tensor) -> np.ndarray:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    fx = {"shape": {"H": H, "I": I, "G": G, "n": N}, "source": "reference wisp/quant.py, wisp/kernels.py"}

    # quantize / dequant, bits 4/3/2, N_EXPERTS experts each (seeds 100*bits + e)
    pools = {}
    fx["quant"] = []
    for bits in (4, 3, 2):
        rows = []
        for e in range(N_EXPERTS):
            seed = 100 * bits + e
            wb = expert_input(seed)
            packed = RQ.quantize(bf16(wb), bits, G).numpy()
            deq = RQ.dequant(torch.from_numpy(packed)[None], N, bits, G)[0]
            d16 = bits16(deq)
            fx["quant"].append(
                {"bits": bits, "seed": seed, "input_sha256": sha(wb), "nbytes": int(packed.size),
                 "packed_sha256": sha(packed), "packed_head": packed[:64].tolist(),
                 "dequant_sha256": sha(d16), "dequant_head": d16.reshape(-1)[:64].tolist()}
            )
            rows.append(packed)
        pools[bits] = torch.from_numpy(np.stack(rows))

    # fused decode layer, k = 3 of the N_EXPERTS experts
    fx["decode"] = []
    for case, (bits, fn) in enumerate([(4, "moe_decode_q4"), (4, "moe_decode_q4_fast"), (3, "moe_decode_q3_fast")]):
        rs = np.random.RandomState(900 + case)
        slots = rs.permutation(N_EXPERTS)[:3].astype(np.int64)
        w = torch.softmax(torch.from_numpy(rs.standard_normal(3).astype(np.float32)), 0)
        xb = x_input(950 + case)
        x = bf16(xb)
        pool = pools[bits]
        if fn == "moe_decode_q4":
            out = RK.moe_decode_q4(pool, torch.from_numpy(slots), x, w, N, H, I)
        else:
            meta = torch.cat([torch.from_numpy(slots).float(), w.float()])
            out = getattr(RK, fn)(pool, meta, x, 3, N, H, I)
        o16 = bits16(out.to(torch.bfloat16))
        fx["decode"].append(
            {"fn": fn, "bits": bits, "slots": slots.tolist(), "weights_f32": w.numpy().tolist(), "x_seed": 950 + case,
             "x_sha256": sha(xb), "out_dtype": str(out.dtype), "out_bf16": o16.tolist()}
        )

    # rope_decode, bf16 and fp32 (q [1,Hq,1,D], k [1,Hk,1,D], cos/sin [1,1,D])
    fx["rope"] = []
    for case, dt in enumerate([torch.bfloat16, torch.float32]):
        hq, hk, d = 4, 2, 64
        rs = np.random.RandomState(700 + case)
        q = torch.from_numpy(rs.standard_normal((1, hq, 1, d)).astype(np.float32)).to(dt)
        k = torch.from_numpy(rs.standard_normal((1, hk, 1, d)).astype(np.float32)).to(dt)
        ang = torch.from_numpy(rs.uniform(-3, 3, d // 2).astype(np.float32))
        emb = torch.cat([ang, ang])
        cos, sin = emb.cos().to(dt).view(1, 1, d), emb.sin().to(dt).view(1, 1, d)
        qo, ko = RK.rope_decode(q, k, cos, sin)

        def raw(t):
            return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).numpy().tolist()

        fx["rope"].append(
            {"dtype": str(dt).replace("torch.", ""), "hq": hq, "hk": hk, "d": d,
             "q": raw(q), "k": raw(k), "cos": raw(cos), "sin": raw(sin), "qo": raw(qo), "ko": raw(ko)}
        )

    with open(OUT, "w") as f:
        json.dump(fx, f, separators=(",", ":"))
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
