"""Write the golden fixtures under tests/golden/.

``reference_kats.json`` holds, as data, the known-answer inputs and expected
outputs that the reference's own CPU tests state for this path. Each entry
names the reference test it comes from (file:line, relative to the local-kimi
repository root). Nothing here imports or runs the reference: the values are
the literal inputs those tests build and the outputs they assert.

``oracle_vectors.npz`` holds small seeded input/output vectors produced by this
repository's oracle. They guard the oracle against drift between edits; the
oracle itself is pinned by the KATs and the mathematical checks in
tests/test_oracle_*.py.

Run: ``python tests/golden/make_golden.py`` from the repository root.
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _sigmoid(v: float) -> float:
    return 1.0 / (1.0 + math.exp(-v))


def reference_kats() -> dict:
    kats: dict = {}

    # test_quant_w4a16.py:22-52 -- grid weight: code pattern (i % 15) - 7 over a
    # 32-wide group, times per-group scales; quantise/dequantise is exact and the
    # recovered scales equal the generating ones.
    kats["codec_grid_round_trip"] = {
        "source": "tests/test_quant_w4a16.py:22-52",
        "group_size": 32,
        "code_pattern": [i % 15 - 7 for i in range(32)],
        "scales": [[0.25, 2.0], [8.0, 0.5]],
        "expect": "dequantise(quantise(w)) == w and scales == generating scales",
    }
    # test_quant_w4a16.py:135-143 -- all-zero tensor: every scale is 1.0.
    kats["codec_zero_tensor"] = {
        "source": "tests/test_quant_w4a16.py:135-143",
        "shape": [3, 64], "group_size": 32, "expected_scale": 1.0,
    }
    # test_w4a16_gemv.py:26-43 -- nibble order, sign and group index.
    nib = [i % 16 for i in range(64)]
    kats["codec_nibble_sign_group"] = {
        "source": "tests/test_w4a16_gemv.py:26-43",
        "group_size": 32,
        "packed": [[nib[2 * j] | (nib[2 * j + 1] << 4) for j in range(32)]],
        "scales": [[1.0, 10.0]],
        "spot_values": {"0": 0.0, "7": 7.0, "8": -8.0, "15": -1.0, "33": 10.0, "40": -80.0},
        "expected": [[(v - 16 if v >= 8 else v) * (1.0 if i < 32 else 10.0)
                      for i, v in enumerate(nib)]],
    }
    # test_w4a16_dense_gemv.py:25-45 -- two rows, second row reversed nibbles.
    first = [i % 16 for i in range(64)]
    second = first[::-1]
    rows = [first, second]
    scales = [[1.0, 10.0], [0.5, 2.0]]
    kats["codec_dense_two_rows"] = {
        "source": "tests/test_w4a16_dense_gemv.py:25-45",
        "group_size": 32,
        "packed": [[r[2 * j] | (r[2 * j + 1] << 4) for j in range(32)] for r in rows],
        "scales": scales,
        "expected": [[(v - 16 if v >= 8 else v) * scales[ri][i // 32] for i, v in enumerate(r)]
                     for ri, r in enumerate(rows)],
        "spot_values": {"0,7": 7.0, "0,8": -8.0, "0,15": -1.0, "0,33": 10.0, "1,0": -0.5},
    }
    # test_w4a16_gemv.py:46-57 and test_moe_swiglu.py:13-34 -- SwiGLU rounding
    # contract: accumulators 1.003 rounded to bf16 before SiLU give a result
    # different from SiLU in fp32 rounded once.
    kats["swiglu_rounding_contract"] = {
        "source": "tests/test_w4a16_gemv.py:46-57; tests/test_moe_swiglu.py:13-34",
        "gate_accumulator": 1.003, "up_accumulator": 1.003,
        "expect": "bf16-first result != fp32-through result",
    }
    # test_moe_combine.py:65-90 -- shared expert added with weight exactly 1.
    kats["combine_shared_weight_one"] = {
        "source": "tests/test_moe_combine.py:65-90",
        "reduction": 32, "group_size": 32,
        "activated_value": 1.0,
        "expert_indices": [[0, 1]],
        "combine_weights": [[0.25, 0.0]],
        "constant_codes": [1, 2], "scales": 1.0,
        "expected": [[72.0]],
    }
    # test_klinear_forward.py:43-75 -- router renormalises the selected sigmoid
    # scores and applies the scaling factor.
    logits = [3.0, 2.0, 1.0, 0.0]
    g = [_sigmoid(logits[0]), _sigmoid(logits[1])]
    kats["router_renorm_scale"] = {
        "source": "tests/test_klinear_forward.py:43-75",
        "router_weight": [[3.0, 0.0], [2.0, 0.0], [1.0, 0.0], [0.0, 0.0]],
        "hidden": [[1.0, 0.0]],
        "top_k": 2, "routed_scaling_factor": 2.446,
        "expected_index_set": [0, 1],
        "expected_weights_for_indices_0_1": [g[0] / sum(g) * 2.446, g[1] / sum(g) * 2.446],
        "expected_weight_sum": 2.446,
    }
    # test_decode_equivalence.py:70-86 -- shape-stable routes append the shared id.
    kats["shape_stable_indices"] = {
        "source": "tests/test_decode_equivalence.py:70-86",
        "expert_indices": [[4, 1, 7], [2, 6, 0]],
        "shared_expert_id": 8,
        "expected": [[4, 1, 7, 8], [2, 6, 0, 8]],
    }
    # test_kernels_mxfp4.py:94-130 -- expert schedule union and counts.
    kats["schedule_union_counts"] = {
        "source": "tests/test_kernels_mxfp4.py:94-111",
        "expert_indices": [[1, 2, 2, -1], [7, 1, -1, -1], [7, 9, 9, 1]],
        "expected_union_size": 4,
        "expected_counts": [[1, 3], [2, 2], [7, 2], [9, 2]],
    }
    kats["schedule_zero_and_duplicate_routes"] = {
        "source": "tests/test_kernels_mxfp4.py:114-130",
        "hidden": [[2.0, -1.0], [3.0, 5.0]],
        "expert_indices": [[-1, -1, -1], [3, 3, -1]],
        "routing_weights": [[0.2, 0.8, 1.0], [0.25, 0.75, 4.0]],
        "expert_fn": "tokens + expert_id",
        "expected_union_size": 1,
        "expected_counts": [[3, 2]],
        "expected_values": [[0.0, 0.0], [6.0, 8.0]],
    }
    # test_k3ref_dequant.py:14-38 -- both nibbles and E8M0 exponents.
    codebook = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    codebook = codebook + [-v for v in codebook]
    fc = list(range(16)) * 2
    sc = list(reversed(range(16))) * 2
    kats["mxfp4_nibbles_and_exponents"] = {
        "source": "tests/test_k3ref_dequant.py:14-38",
        "packed": [[fc[2 * j] | (fc[2 * j + 1] << 4) for j in range(16)],
                   [sc[2 * j] | (sc[2 * j + 1] << 4) for j in range(16)]],
        "scale": [[128], [126]],
        "expected": [[codebook[c] * 2.0 for c in fc], [codebook[c] * 0.5 for c in sc]],
    }
    # test_dequant_codec.py:11-113 -- hand-built buffer, bit exact, -0.0 kept.
    packed = [0x80, 0x91, 0xA2, 0xB3, 0xC4, 0xD5, 0xE6, 0xF7,
              0x08, 0x19, 0x2A, 0x3B, 0x4C, 0x5D, 0x6E, 0x7F]
    codes = [0, 8, 1, 9, 2, 10, 3, 11, 4, 12, 5, 13, 6, 14, 7, 15,
             8, 0, 9, 1, 10, 2, 11, 3, 12, 4, 13, 5, 14, 6, 15, 7]
    expected = [codebook[c] * 2.0 for c in codes]
    kats["mxfp4_hand_built_buffer"] = {
        "source": "tests/test_dequant_codec.py:11-113",
        "packed": [packed], "scale": [[128]],
        "expected_codes": codes,
        "expected": [expected],
        "expected_float32_bits": [[int(np.array(v, dtype=np.float32).view(np.uint32)) for v in expected]],
        "negative_zero_positions": [1, 16],
    }
    # test_kernels_mxfp4.py:31-44 -- unfused reference vs canonical decoder.
    first = list(range(16)) * 4
    second = list(reversed(range(16))) * 4
    kats["mxfp4_two_groups"] = {
        "source": "tests/test_kernels_mxfp4.py:31-44",
        "packed": [[first[2 * j] | (first[2 * j + 1] << 4) for j in range(32)],
                   [second[2 * j] | (second[2 * j + 1] << 4) for j in range(32)]],
        "scale": [[126, 130], [127, 125]],
        "spot_values": {"0,0": 0.0, "0,1": 0.25, "0,32": 0.0, "0,33": 4.0},
    }
    # quant/verify.py:165-176 -- the negative-control probe (exact on its grid),
    # against which the three broken decoders of verify.py:140-162 must fail.
    kats["negative_control_probe"] = {
        "source": "engine/quant/verify.py:140-176",
        "group_size": 32,
        "code_pattern": [i % 15 - 7 for i in range(32)],
        "scales": [[0.25, 2.0], [8.0, 0.5]],
        "broken_decoders": ["wrong_group_axis", "wrong_scale", "swapped_nibbles"],
    }
    return kats


def oracle_vectors() -> dict:
    sys.path.insert(0, ROOT)
    from oracle import moe as M
    from oracle import mxfp4 as X
    from oracle import w4a16 as W
    from oracle.bf16 import f32_to_bf16_bits

    rng = np.random.default_rng(20260729)
    out: dict = {}
    for g in (32, 128):
        n, k = 96, 256
        w = f32_to_bf16_bits(rng.normal(0, 0.02, (n, k)).astype(np.float32))
        p, s = W.quantise(w, g)
        x = f32_to_bf16_bits(rng.normal(0, 1, (2, k)).astype(np.float32))
        out[f"dense_g{g}_w"] = w
        out[f"dense_g{g}_packed"] = p
        out[f"dense_g{g}_scales"] = s
        out[f"dense_g{g}_x"] = x
        out[f"dense_g{g}_y"] = W.dense(x, p, s, g)
    # small MoE block: 6 routed + 1 shared expert, top-2, hidden 256, inter 128
    e, h, i, g = 7, 256, 128, 128
    def bank(nr, kr):
        ps, ss = [], []
        for _ in range(e):
            wb = f32_to_bf16_bits(rng.normal(0, 0.02, (nr, kr)).astype(np.float32))
            pp, sss = W.quantise(wb, g)
            ps.append(pp)
            ss.append(sss)
        return np.stack(ps), np.stack(ss)
    w1p, w1s = bank(i, h)
    w3p, w3s = bank(i, h)
    w2p, w2s = bank(h, i)
    x = f32_to_bf16_bits(rng.normal(0, 1, (3, h)).astype(np.float32))
    logits = rng.normal(0, 1, (3, e - 1)).astype(np.float32)
    y, idx, wts = M.moe_block(x, logits, None, w1p, w1s, w3p, w3s, w2p, w2s, top_k=2,
                              routed_scaling_factor=2.446, group_size=g)
    out.update(moe_x=x, moe_logits=logits, moe_w1p=w1p, moe_w1s=w1s, moe_w3p=w3p, moe_w3s=w3s,
               moe_w2p=w2p, moe_w2s=w2s, moe_y=y, moe_idx=idx, moe_w=wts)
    wf = rng.normal(0, 0.02, (48, 64)).astype(np.float32)
    mp, ms = X.quantize(wf)
    xm = f32_to_bf16_bits(rng.normal(0, 1, (5, 64)).astype(np.float32))
    out.update(mx_w=wf, mx_packed=mp, mx_scale=ms, mx_x=xm, mx_y=X.linear(xm, mp, ms))
    return out


def main() -> None:
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1, sort_keys=True)
        f.write("\n")
    np.savez_compressed(os.path.join(HERE, "oracle_vectors.npz"), **oracle_vectors())
    print("wrote reference_kats.json and oracle_vectors.npz")


if __name__ == "__main__":
    main()
