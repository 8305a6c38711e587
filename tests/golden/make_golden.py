"""Writes the golden fixtures of the quantized GEMV path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no vectors for this path (no kernel tests beyond kernel
names, qw35-server/src/tests/metal_bridge.rs:1-15), so these fixtures are
produced by this repository's oracle, whose formulas are pinned independently
by tests/test_oracle_*.py (closed forms, exhaustive tables, hand-computed words).
They freeze the oracle's outputs so that any later change to it, or to the HIP
library that consumes them (tests/test_gpu_gemv.py::test_golden_fixtures), is caught.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import gf4, q4_k, q8_0  # noqa: E402
from oracle import matvec as om  # noqa: E402


def main() -> None:
    rng = np.random.default_rng(20261201)
    out = {}
    # GF4: weights bf16(0.02 N(0,1)) packed, plus arbitrary words
    w = om.bf16_round((rng.standard_normal((32, 512)) * 0.02).astype(np.float32))
    out["gf4_words"] = gf4.gf4_pack(w)
    out["gf4_deq"] = gf4.gf4_dequant(out["gf4_words"])
    x = rng.standard_normal((2, 512)).astype(np.float32)
    a = rng.uniform(0.5, 2.0, 512).astype(np.float32)
    out["x"] = x
    out["awq"] = a
    out["gf4_y"] = om.matvec_f64(out["gf4_deq"], x, a)
    words = rng.integers(0, 2**32, (8, 64), dtype=np.uint64).astype(np.uint32)
    b = words & np.uint32(0xFF)
    words = np.where(((b >> np.uint32(2)) & np.uint32(0x1F)) == np.uint32(0x1F), words & np.uint32(0xFFFFFF83), words)
    out["gf4_any_words"] = words.astype(np.uint32)
    out["gf4_any_deq"] = gf4.gf4_dequant(out["gf4_any_words"])
    # q8_0 and Q4_K
    w8 = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    out["q8_0_raw"] = q8_0.q8_0_quantize(w8)
    out["q8_0_deq"] = q8_0.q8_0_dequant(out["q8_0_raw"])
    out["q8_0_y"] = om.matvec_f64(out["q8_0_deq"], x, a)
    w4 = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    out["q4_k_raw"] = q4_k.q4_k_quantize(w4)
    out["q4_k_deq"] = q4_k.q4_k_dequant(out["q4_k_raw"])
    out["q4_k_y"] = om.matvec_f64(out["q4_k_deq"], x, a)
    # e5m2 table
    out["e5m2_table"] = gf4.e5m2_byte_to_fp32(np.arange(256, dtype=np.uint8))
    np.savez_compressed(os.path.join(HERE, "gemv_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "gemv_golden.npz"))


if __name__ == "__main__":
    main()
