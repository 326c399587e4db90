"""Writes ternary_blocks.json: the 128-weight block known answers of the
reference's own tests (test/gguf.test.ts:32-124), as data.

  - Q1_0: binary16 scale 1.5 (0x3e00), every sign byte 0xaa: weights
    alternate -1.5, +1.5.
  - PQ2_0: scale 0.5 (0x3800), every code byte 0x64 (codes 0, 1, 2, 1):
    weights repeat -0.5, 0, 0.5, 0.
  - PTQ1_0: the trits t_i = ((7 i + 3) mod 3) - 1 with scale 2.0 (0x4000),
    packed by the test's encoder (five trits per byte in base 3, most
    significant first, then q -> floor((256 q + 242) / 243); the two tail
    bytes hold four trits and one factor 3): weights 2 t_i.
  - Q4_0 / Q4_1 (32 weights): the same test's blocks.

Run from the repository root: python tests/golden/make_ternary_blocks.py
"""
import json
import os


def ptq1_encode(trits, scale_bits):
    block = [0] * 28
    block[26], block[27] = scale_bits & 0xFF, scale_bits >> 8

    def pack(idx, extra_factor):
        q = 0
        for i in idx:
            q = q * 3 + (trits[i] + 1)
        q *= extra_factor
        return (q * 256 + 242) // 243

    for m in range(16):                       # weights m + 16 n
        block[m] = pack([m + 16 * n for n in range(5)], 1)
    for m in range(8):                        # weights 80 + m + 8 n
        block[16 + m] = pack([80 + m + 8 * n for n in range(5)], 1)
    for h in range(2):                        # weights 120 + h + 2 n
        block[24 + h] = pack([120 + h + 2 * n for n in range(4)], 3)
    return block


def main():
    trits = [((i * 7 + 3) % 3) - 1 for i in range(128)]
    cases = [
        {"name": "q1_0_alternating_signs", "type": 41,
         "block": [0x00, 0x3e] + [0xaa] * 16,
         "weights": [1.5 if j % 2 == 1 else -1.5 for j in range(128)]},
        {"name": "pq2_0_code_pattern", "type": 142,
         "block": [0x00, 0x38] + [0x64] * 32,
         "weights": [[-0.5, 0.0, 0.5, 0.0][j % 4] for j in range(128)]},
        {"name": "ptq1_0_round_trip", "type": 143,
         "block": ptq1_encode(trits, 0x4000),
         "weights": [2.0 * t for t in trits]},
        {"name": "q4_0_nibbles", "type": 2,
         "block": [0x00, 0x38] + [0x97] * 16,
         "weights": [-0.5] * 16 + [0.5] * 16},
        {"name": "q4_1_nibbles_and_min", "type": 3,
         "block": [0x00, 0x38, 0x00, 0x3c] + [0x42] * 16,
         "weights": [2.0] * 16 + [3.0] * 16},
    ]
    out = {"about": "Block known answers of test/gguf.test.ts:32-124 (dequantizeBlock128Cpu, "
                    "dequantizeBlockCpu); written by make_ternary_blocks.py.",
           "cases": cases}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ternary_blocks.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
