"""Writes the NF4 golden fixtures in this directory.

These vectors are SELF-GENERATED from this repository's CPU oracle
(oracle/nf4_oracle.py): the reference ships no NF4 golden vectors and its NF4
arithmetic lives in bitsandbytes, which is neither vendored nor installed. They
freeze the oracle's output so later changes to it (or to the kernels) are caught.

Inputs follow the benchmark recipe: torch.Generator().manual_seed(seed),
randn(...) * std, cast to the source dtype.

Run:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import nf4_oracle as O  # noqa: E402


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def as_np(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16), O.DT_BF16
    if t.dtype == torch.float16:
        return t.numpy(), O.DT_F16
    return t.numpy(), O.DT_F32


def edge_input():
    """fp32 vector whose blocks hit the decision boundaries exactly.

    Block b (64 elements) starts with 1.0, so absmax = 1 and s = x exactly; the
    rest are each rule's 15 boundaries and their fp32 neighbours. Then a zero
    block, a block of +-absmax / 0, and a block of tiny values.
    """
    vals = []
    for rule in O.ROUNDINGS:
        b = O.decision_boundaries(rule)
        blk = [np.float32(1.0)]
        for v in b:
            blk += [np.nextafter(v, np.float32(-2)), v, np.nextafter(v, np.float32(2))]
        blk += [np.float32(0)] * (64 - len(blk))
        vals += blk[:64]
        blk = [np.float32(-1.0)] + list(O.midpoint_thresholds()) + list(-O.midpoint_thresholds())
        blk += [np.float32(0)] * (64 - len(blk))
        vals += blk[:64]
    vals += [np.float32(0)] * 64                                    # all-zero block
    vals += [np.float32(0.02), np.float32(-0.02), np.float32(0)] * 21 + [np.float32(0.02)]
    vals += list((np.arange(64, dtype=np.float32) - 31.5) * np.float32(1e-30))  # tiny, fp32 only
    return np.array(vals, dtype=np.float32)


def main():
    cases = {
        "nf4_f16_64x128_bs64": (seeded((64, 128), 1234, 0.02, torch.float16), 64),
        "nf4_bf16_64x128_bs64": (seeded((64, 128), 1235, 0.02, torch.bfloat16), 64),
        "nf4_f32_48x64_bs128": (seeded((48, 64), 1236, 1.0, torch.float32), 128),
        "nf4_f16_odd1001_bs64": (seeded((1001,), 1237, 0.02, torch.float16), 64),
        "nf4_f32_edge_bs64": (torch.from_numpy(edge_input()), 64),
    }
    for name, (x, bs) in cases.items():
        xn, tag = as_np(x)
        out = {"x": xn, "dtype_tag": np.int32(tag), "blocksize": np.int32(bs)}
        for rule in O.ROUNDINGS:
            packed, absmax, codes = O.quantize(xn, tag, bs, rule)
            out[f"packed_{rule}"] = packed
            out[f"absmax_{rule}"] = absmax
        n = xn.size
        out["deq_f16"] = O.dequantize(out["packed_argmin"], out["absmax_argmin"], n, bs, O.DT_F16).view(np.uint16)
        out["deq_bf16"] = O.dequantize(out["packed_argmin"], out["absmax_argmin"], n, bs, O.DT_BF16)
        out["deq_f32"] = O.dequantize(out["packed_argmin"], out["absmax_argmin"], n, bs, O.DT_F32)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
        dis = int((out["packed_argmin"] != out["packed_threshold"]).sum())
        print(f"{name}: n={n} blocksize={bs} bytes differing between rules={dis}")


if __name__ == "__main__":
    main()
