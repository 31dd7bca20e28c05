"""Writes tests/golden/kats.json: known answers for the oracle, from closed forms.

Nothing here calls the oracle or the reference (the reference is Rust and
cannot run in this image).  The cases restate the reference tests'
assertions (crates/mrml-tensor/tests/quant_test.rs:24-57,
examples/cuda_prefill_primitives.rs:23-49) with exact expected values worked
out by hand:
  * f16 truncation of 1/127, 100/127, 2.5/127 (quant.rs:81-104);
  * Q4_0 x Q8_0 dots whose activations quantise exactly (amax = 127 gives
    scale 1, so q = x) or to the all-ones case (q = 127, d = 0x2008);
  * Q8_0 quantiser bytes for all-ones and for round-half-away-from-zero ties.
Run:  python tests/golden/make_kats.py
"""
import json
from pathlib import Path


def q4_block(d_bits, byte):
    return [d_bits & 0xFF, d_bits >> 8] + [byte] * 16


def main():
    exact_x = [127] + [((i * 37) % 255) - 127 for i in range(1, 32)]   # integers, amax 127
    kats = {
        "f32_to_f16_trunc": [
            {"x": 1 / 127, "h": 0x2008},
            {"x": 100 / 127, "h": 0x3A4C},
            {"x": 2.5 / 127, "h": 0x250A},
            {"x": 1.0, "h": 0x3C00},
            {"x": 65504.0, "h": 0x7BFF},
            {"x": 1e6, "h": 0x7C00},
            {"x": 1e-6, "h": 0x0000},
        ],
        "q4_0_dot": [
            # quant_test.rs:42-57: d_w = 1, weights +1, activations Q8_0(1) -> q=127, d_a=f16(0x2008)
            {"name": "0x99_ones", "w": q4_block(0x3C00, 0x99), "x": [1.0] * 32, "y": 4064 * 129 / 16384},
            # quant_test.rs:24-40: 0x88 -> all weights 0
            {"name": "0x88_zero", "w": q4_block(0x3C00, 0x88), "x": [float(v) for v in exact_x], "y": 0.0},
            # cuda_prefill_primitives.rs:23-49 closed forms, exact activations
            {"name": "0x98_upper", "w": q4_block(0x3C00, 0x98), "x": [float(v) for v in exact_x],
             "y": float(sum(exact_x[16:]))},
            {"name": "0x87_lower", "w": q4_block(0x3C00, 0x87), "x": [float(v) for v in exact_x],
             "y": float(-sum(exact_x[:16]))},
            # d_w = 0.5 (0x3800), weights -8 (nibble 0) everywhere
            {"name": "0x00_min", "w": q4_block(0x3800, 0x00), "x": [float(v) for v in exact_x],
             "y": -8 * 0.5 * float(sum(exact_x))},
        ],
        "q8_0_quantize": [
            {"name": "ones", "x": [1.0] * 32, "bytes": [0x08, 0x20] + [127] * 32},
            {"name": "ties", "x": [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5] + [0.0] * 25,
             "bytes": [0x00, 0x3C, 127, 3, 253, 1, 255, 2, 254] + [0] * 25},
            {"name": "zeros", "x": [0.0] * 32, "bytes": [0] * 34},
        ],
    }
    out = Path(__file__).resolve().parent / "kats.json"
    out.write_text(json.dumps(kats, indent=1) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
