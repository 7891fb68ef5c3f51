"""Writes reference_kats.json: the known-answer tests the reference's own test
suite holds for this path, as data (inputs, expected outputs, bounds).

Provenance (eclipse005/qwen3-aligner-wgpu):
  bf16_known_answer          src/half16.rs:113-119 (0.1f32 -> 0x3DCD, not the
                             truncated 0x3DCC)
  round_trip_values          src/half16.rs:99-110
  bf16_halfway_grid          src/shaders.rs:219-232 (exponent x mantissa-top x
                             low-16-bits x sign)
  bf16_sweep                 src/shaders.rs:234-239 (LCG s = s*1664525 +
                             1013904223 from 0x12345678, 500 000 draws, > 400 000
                             finite values checked)
  gemm_row_major_matches_naive
                             src/cpu_decoder.rs:620-646 (shapes, closed-form
                             inputs x[i] = (i*13 % 61)*0.03 - 0.9,
                             w[i] = (i*7 % 53)*0.02 - 0.5, worst |d| < 1e-3)
The reference is Rust and cannot be built or run here; these are the values
its tests state.  Run: python tests/golden/make_reference_kats.py
"""
import json
import os

KATS = {
    "bf16_known_answer": {"input": 0.1, "bits": 0x3DCD},
    "round_trip_values": [0.0, 1.0, -1.0, 0.1, 3.14159, 1e-5, 6.5e4, -2.5e-3],
    "bf16_halfway_grid": {
        "exponents": [0, 1, 2, 50, 63, 64, 100, 126, 127, 128, 200, 250, 253, 254],
        "mantissa_top": [0, 1, 2, 0x3F, 0x40, 0x7E, 0x7F],
        "low_bits": [0, 1, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xFFFE, 0xFFFF],
    },
    "bf16_sweep": {"seed": 0x12345678, "count": 500000, "min_checked": 400000},
    "gemm_row_major_matches_naive": {
        "shapes": [[3, 5, 4], [8, 8, 8], [4, 64, 32], [210, 1280, 1024], [64, 3072, 1024],
                   [64, 1024, 3072]],
        "x": {"mul": 13, "mod": 61, "scale": 0.03, "offset": 0.9},
        "w": {"mul": 7, "mod": 53, "scale": 0.02, "offset": 0.5},
        "bound": 1e-3,
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(out, "w") as f:
        json.dump(KATS, f, indent=1)
        f.write("\n")
    print("wrote", out)
