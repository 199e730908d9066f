"""Write tests/golden/fp8_golden.json: fp8 known-answer vectors.

The reference holds no golden vectors for tt.fp_to_fp (its only fp8 tests are
Blackwell stochastic-rounding sanity checks, test_tlx.py:5125-5371).  These
vectors come from an independent implementation, PyTorch's CPU float8 dtypes
(round to nearest even, non-saturating: overflow -> NaN for e4m3fn, Inf for
e5m2), used here as a library cross-check only:

  decode[fmt]      fp32 bits of all 256 codes (NaN codes kept as PyTorch's bits;
                   tests compare NaN codes by NaN-ness and sign)
  encode_inputs    fp32 bit patterns: specials, every fp8 value, every midpoint
                   between neighbouring fp8 values (ties) and +-1 ulp around it,
                   overflow boundaries, and seeded random patterns
  encode[fmt]      PyTorch's code for each input (non-saturating)
  encode_sat[fmt]  PyTorch's code for clamp(x, -max, max) (NaN kept), the
                   reference's saturating idiom (mxfp8_utils.py:36-38)

Run: python tests/golden/make_fp8_golden.py
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FMTS = {"e4m3fn": (torch.float8_e4m3fn, 448.0), "e5m2": (torch.float8_e5m2, 57344.0)}


def decode_table(td):
    codes = torch.arange(256, dtype=torch.uint8)
    return codes.view(td).float().view(torch.int32).numpy().view(np.uint32)


def inputs():
    bits = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000,
            0x7F800001, 0xFFBFFFFF, 0x00000001, 0x007FFFFF, 0x80000001, 0x807FFFFF,
            0x00800000, 0x80800000, 0x7F7FFFFF, 0xFF7FFFFF]
    for td, fmax in FMTS.values():
        vals = torch.arange(256, dtype=torch.uint8).view(td).float().numpy()
        fin = np.sort(np.unique(np.abs(vals[np.isfinite(vals)])))
        # every value, every midpoint, midpoint +- 1 ulp, both signs
        mids = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
        # the virtual next value above max (its midpoint decides overflow)
        nxt = np.float32(2 * fin[-1] - fin[-2])
        extra = np.array([(fin[-1] + np.float64(nxt)) / 2, nxt, 2 * nxt], dtype=np.float32)
        pts = np.concatenate([fin, mids, extra]).astype(np.float32)
        b = pts.view(np.uint32)
        allb = np.concatenate([b, b + 1, b - 1])
        allb = allb[(allb & 0x7FFFFFFF) <= 0x7F800000]
        bits += list(allb) + list(allb | 0x80000000)
    g = np.random.default_rng(20261201)
    bits += list(g.integers(0, 1 << 32, size=4096, dtype=np.uint64).astype(np.uint32))
    return np.unique(np.array(bits, dtype=np.uint32))


def main():
    x_bits = inputs()
    x = x_bits.view(np.float32)
    out = {"encode_inputs": [int(v) for v in x_bits], "decode": {}, "encode": {},
           "encode_sat": {}}
    for name, (td, fmax) in FMTS.items():
        out["decode"][name] = [int(v) for v in decode_table(td)]
        t = torch.from_numpy(x.copy())
        out["encode"][name] = t.to(td).view(torch.uint8).numpy().tolist()
        clamped = torch.where(torch.isnan(t), t, t.clamp(-fmax, fmax))
        out["encode_sat"][name] = clamped.to(td).view(torch.uint8).numpy().tolist()
    path = os.path.join(HERE, "fp8_golden.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {path}: {len(x_bits)} encode inputs")


if __name__ == "__main__":
    main()
