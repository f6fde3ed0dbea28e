"""Writes tests/golden/reference_kats.json: the known-answer vectors that the
reference's own unit tests pin for this path, restated as data.

Every entry names the reference test it comes from.  Inputs are the bytes /
values those tests construct; expected outputs are the literals those tests
assert.  No reference code is run (the reference is Zig and cannot be built
here); this script only serialises the literals.

    python tests/golden/make_golden.py
"""
import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(x: float) -> int:
    return struct.unpack("<H", struct.pack("<e", x))[0]


def q4k_block():
    # src/gguf/ggml.zig:1938-1966 "q4_k dequant with handcrafted block"
    blk = bytearray(144)
    blk[0:2] = struct.pack("<H", f16_bits(1.0))  # d
    blk[2:4] = struct.pack("<H", f16_bits(0.0))  # dmin
    for i in range(4):  # scales[0..4] = 1 (sc = 1 for sub-blocks 0..3)
        blk[4 + i] = 1
    for i in range(16, 144):
        blk[i] = 0x31  # low nibble 1, high nibble 3
    return {
        "source": "src/gguf/ggml.zig:1938-1966",
        "block_hex": blk.hex(),
        "expect_vals": {"0": 1.0, "32": 3.0, "64": 1.0, "96": 3.0, "128": 0.0, "255": 0.0},
        "expect_dot_ones": 256.0,
        "dot_tol": 1e-2,
    }


def q6k_block():
    # src/gguf/ggml.zig:1968-1977 "q6_k dequant with handcrafted block"
    blk = bytearray(210)
    for i in range(192, 208):
        blk[i] = 1  # all 16 scales = 1
    blk[208:210] = struct.pack("<H", f16_bits(0.5))
    return {"source": "src/gguf/ggml.zig:1968-1977", "block_hex": blk.hex(), "expect_all": -16.0}


def route_cases():
    return [
        {
            # src/gguf/moe.zig:210-223
            "source": "src/gguf/moe.zig:210-223",
            "logits": [0.0, 1.0, 2.0, 3.0],
            "bias": [10.0, 0.0, 0.0, 0.0],
            "n_used": 2,
            "gating": "sigmoid",
            "weights_norm": False,
            "weights_scale": 1.0,
            "expect_ids": [0, 3],
            "expect_gates": "sigmoid(0), sigmoid(3)",
            "gate_tol": 1e-6,
        },
        {
            # src/gguf/moe.zig:225-242
            "source": "src/gguf/moe.zig:225-242",
            "logits": [0.5, 3.0, 1.0, 2.0],
            "bias": None,
            "n_used": 2,
            "gating": "softmax_topk",
            "weights_norm": False,
            "weights_scale": 1.0,
            "expect_ids": [1, 3],
            "expect_gates": "exp(3)/(exp(3)+exp(2)), exp(2)/(exp(3)+exp(2))",
            "gate_tol": 1e-6,
        },
        {
            # src/gguf/moe.zig:244-258 (renormalised top-2 sums to one)
            "source": "src/gguf/moe.zig:244-258",
            "logits": [1.0, 2.0, 3.0, 4.0],
            "bias": None,
            "n_used": 2,
            "gating": "softmax",
            "weights_norm": True,
            "weights_scale": 1.0,
            "expect_gate_sum": 1.0,
            "gate_tol": 1e-6,
        },
        {
            # src/gguf/moe.zig:244-258 (without renorm the raw top-2 mass < 0.95)
            "source": "src/gguf/moe.zig:244-258",
            "logits": [1.0, 2.0, 3.0, 4.0],
            "bias": None,
            "n_used": 2,
            "gating": "softmax",
            "weights_norm": False,
            "weights_scale": 1.0,
            "expect_gate_sum_below": 0.95,
        },
        {
            # src/gguf/moe.zig:260-267
            "source": "src/gguf/moe.zig:260-267",
            "logits": [1.0, 2.0, 3.0, 4.0],
            "bias": None,
            "n_used": 2,
            "gating": "softmax",
            "weights_norm": True,
            "weights_scale": 2.5,
            "expect_gate_sum": 2.5,
            "gate_tol": 1e-5,
        },
    ]


def hottest():
    # src/core/stats.zig:161-171
    return {
        "source": "src/core/stats.zig:161-171",
        "counts": [1, 100, 5, 100, 0, 50],
        "expert_bytes": 10,
        "budget": 20,
        "expect_ids_set": [1, 3],
    }


def lru():
    # src/engine/expert_cache.zig:258-279: capacity 2; reserve 10, 11; find 10
    # (11 becomes LRU); reserve 12 evicts 11.
    return {
        "source": "src/engine/expert_cache.zig:258-279",
        "capacity": 2,
        "ops": [["reserve", 10], ["reserve", 11], ["find", 10, True], ["reserve", 12],
                ["find", 11, False], ["find", 10, True], ["find", 12, True]],
    }


def nonfinite():
    # src/gguf/ggml.zig:2188-2210: x[i] = i % 7 over 64 values with NaN, +Inf,
    # -Inf at 0..2; every block scale finite and every q in [-127, 127]; an
    # all-NaN block gives d = 0 and q = 0.
    x = [float(i % 7) for i in range(64)]
    return {
        "source": "src/gguf/ggml.zig:2188-2210",
        "x": ["nan", "inf", "-inf"] + x[3:],
        "expect_blocks": 2,
    }


def main():
    out = {
        "q4_k_handcrafted": q4k_block(),
        "q6_k_handcrafted": q6k_block(),
        "route": route_cases(),
        "hottest_within_budget": hottest(),
        "lru_eviction": lru(),
        "nonfinite_quantizer": nonfinite(),
        "matvec_tolerances": {
            "source": "src/gguf/ggml.zig:2021-2087",
            "int8_kernel_tol_mass_fraction": 0.01,
            "f16_exponent_bit_clear_mask": 0xFB,
        },
        "q4_0_q8_0_vs_f32": {
            "source": "src/gguf/ggml.zig:1906-1936",
            "rows": 4,
            "cols": 64,
            "q4_0_abs_tol": 0.6,
            "q8_0_abs_tol": 0.05,
        },
    }
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
