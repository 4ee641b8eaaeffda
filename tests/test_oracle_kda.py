"""Pins for oracle/kda.py: the reference's hand-computed cases, closed forms,
invariants of the delta rule, and planted mistakes that those pins catch.

Hand-computed data restated from tests/test_kda_step.py:13-90 and
tests/test_kda_prepare.py:26-123 of the reference (inputs and expected outputs
only)."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import kda as K

# tests/test_kda_step.py:13-90: batch 1, two heads of 4x4 state, scale 0.25
STEP_STATE = np.array([[[[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]],
                        [[2, 0, 1, -1], [1, 3, -2, 4], [0, 5, 2, 1], [4, -1, 0, 2]]]], np.float32)
STEP_Q = np.array([[[1, -1, 0, 0], [0, 1, 0, -1]]], np.float32)
STEP_K = np.array([[[1, 1, 0, 0], [0, 1, 0, 1]]], np.float32)
STEP_V = np.array([[[4.5, 7.0, 9.5, 12.0], [7.0, -1.0, 2.0, 4.0]]], np.float32)
STEP_DECAY_FACTORS = np.array([[[1.0, 0.5, 2.0, 0.25], [0.5, 1.0, 0.25, 2.0]]], np.float32)
STEP_BETA = np.array([[0.5, 0.25]], np.float32)
STEP_EXPECTED_STATE = np.array(
    [[[[1.5, 3.0, 4.5, 6.0], [3.0, 4.0, 5.0, 6.0], [18.0, 20.0, 22.0, 24.0], [3.25, 3.5, 3.75, 4.0]],
      [[1.0, 0.0, 0.5, -0.5], [0.5, 2.5, -1.0, 3.0], [0.0, 1.25, 0.5, 0.25], [7.5, -2.5, 1.0, 3.0]]]],
    np.float32)
STEP_EXPECTED_OUT = np.array([[[-0.375, -0.25, -0.125, 0.0], [-1.75, 1.25, -0.5, 0.0]]], np.float32)


def _step_kat(step=K.decode_step):
    return step(STEP_STATE, STEP_Q, STEP_K, STEP_V, np.log(STEP_DECAY_FACTORS.astype(np.float64)),
                STEP_BETA, 0.25)


def test_decode_step_hand_computed_case():
    state, out = _step_kat()
    np.testing.assert_allclose(state, STEP_EXPECTED_STATE, atol=1e-12, rtol=0)
    np.testing.assert_allclose(out, STEP_EXPECTED_OUT, atol=1e-12, rtol=0)


def test_decode_step_delta_rule_recalls_the_written_value():
    """No decay, beta = 1 and a unit key: afterwards the state maps k exactly
    to v (S'^T k = S^T k + (v - S^T k) |k|^2 = v)."""
    rng = np.random.default_rng(1)
    s = rng.normal(0, 1, (2, 3, 16, 8))
    k = rng.normal(0, 1, (2, 3, 16))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(0, 1, (2, 3, 8))
    state, out = K.decode_step(s, k, k, v, np.zeros((2, 3, 16)), np.ones((2, 3)), 1.0)
    np.testing.assert_allclose(np.einsum("bhkv,bhk->bhv", state, k), v, atol=1e-12)
    np.testing.assert_allclose(out, v, atol=1e-12)  # q = k, scale 1


def test_decode_step_without_beta_only_decays():
    rng = np.random.default_rng(2)
    s = rng.normal(0, 1, (1, 2, 8, 8))
    q, k = rng.normal(0, 1, (2, 1, 2, 8))
    v = rng.normal(0, 1, (1, 2, 8))
    d = -rng.uniform(0, 1, (1, 2, 8))
    state, out = K.decode_step(s, q, k, v, d, np.zeros((1, 2)), 0.5)
    want = s * np.exp(d)[..., None]
    np.testing.assert_allclose(state, want, atol=1e-14)
    np.testing.assert_allclose(out, np.einsum("bhkv,bhk->bhv", want, q * 0.5), atol=1e-14)


def test_decode_step_output_is_linear_in_q():
    rng = np.random.default_rng(3)
    s = rng.normal(0, 1, (1, 1, 8, 4))
    q1, q2, k = rng.normal(0, 1, (3, 1, 1, 8))
    v = rng.normal(0, 1, (1, 1, 4))
    d = -rng.uniform(0, 1, (1, 1, 8))
    b = np.full((1, 1), 0.3)
    _, o1 = K.decode_step(s, q1, k, v, d, b, 0.7)
    _, o2 = K.decode_step(s, q2, k, v, d, b, 0.7)
    _, o12 = K.decode_step(s, q1 + q2, k, v, d, b, 0.7)
    np.testing.assert_allclose(o12, o1 + o2, atol=1e-12)


def _transposed_prediction(state, q, k, v, decay, beta, scale):
    """A plausible mistake: the prediction contracts the value axis (S k, not S^T k)."""
    s = np.asarray(state, np.float64) * np.exp(np.asarray(decay, np.float64))[..., :, None]
    pred = np.einsum("bhkv,bhv->bhk", s, np.asarray(k, np.float64))
    delta = np.asarray(v, np.float64) - pred
    s = s + np.asarray(beta, np.float64)[..., None, None] * np.asarray(k, np.float64)[..., :, None] * delta[..., None, :]
    return s, np.einsum("bhkv,bhk->bhv", s, np.asarray(q, np.float64) * scale)


def _decay_on_value_axis(state, q, k, v, decay, beta, scale):
    """A plausible mistake: the decay scales the value axis instead of the key axis."""
    s = np.asarray(state, np.float64) * np.exp(np.asarray(decay, np.float64))[..., None, :]
    return K.decode_step(s, q, k, v, np.zeros_like(np.asarray(decay, np.float64)), beta, scale)


def _beta_dropped(state, q, k, v, decay, beta, scale):
    return K.decode_step(state, q, k, v, decay, np.ones_like(np.asarray(beta)), scale)


@pytest.mark.parametrize("mistake", [_transposed_prediction, _decay_on_value_axis, _beta_dropped])
def test_planted_step_mistakes_fail_the_hand_computed_case(mistake):
    state, out = _step_kat(mistake)
    assert not (np.allclose(state, STEP_EXPECTED_STATE, atol=1e-6)
                and np.allclose(out, STEP_EXPECTED_OUT, atol=1e-6))


# tests/test_kda_prepare.py:26-58
def test_short_conv_hand_computed_case():
    ins = [np.array([[[5.0]]]), np.array([[[0.0]]]), np.array([[[6.0]]])]
    states = [np.array([[[1.0, 2.0, 3.0, 4.0]]]), np.array([[[4.0, 3.0, 2.0, 1.0]]]),
              np.array([[[-1.0, -2.0, -3.0, -4.0]]])]
    weights = [np.array([[[1.0, 0.0, 0.0, 0.0]]]), np.array([[[0.0, 0.0, 1.0, 0.0]]]),
               np.array([[[1.0, 1.0, 1.0, 1.0]]])]
    outs, new_states = K.short_conv_triple(*ins, *states, *weights, "float32")
    silu = lambda x: x / (1.0 + math.exp(-x))  # noqa: E731
    for o, want in zip(outs, (silu(2.0), silu(1.0), silu(-3.0))):
        assert abs(o.item() - want) < 1e-6
    assert np.array_equal(new_states[0], [[[2.0, 3.0, 4.0, 5.0]]])
    assert np.array_equal(new_states[1], [[[3.0, 2.0, 1.0, 0.0]]])
    assert np.array_equal(new_states[2], [[[-2.0, -3.0, -4.0, 6.0]]])


def test_short_conv_matches_a_loop_and_both_weight_layouts():
    rng = np.random.default_rng(4)
    b, c = 3, 37
    x = rng.normal(0, 1, (b, 1, c))
    st = rng.normal(0, 1, (b, c, 4))
    w = rng.normal(0, 0.5, (c, 4))
    out, ns = K.short_conv(x, st, w, "float32")
    out3, ns3 = K.short_conv(x, st, w[:, None, :], "float32")
    assert np.array_equal(out, out3) and np.array_equal(ns, ns3)
    for bi in range(b):
        for ci in range(c):
            win = [st[bi, ci, 1], st[bi, ci, 2], st[bi, ci, 3], x[bi, 0, ci]]
            conv = sum(win[j] * w[ci, j] for j in range(4))
            want = np.float32(conv / (1.0 + math.exp(-conv)))
            assert out[bi, 0, ci] == want
            assert list(ns[bi, ci]) == win


def test_short_conv_rounds_to_the_storage_dtype():
    x = np.array([[[1.0 + 2.0 ** -9]]])
    st = np.zeros((1, 1, 4))
    w = np.array([[0.0, 0.0, 0.0, 1.0]])
    want = (1.0 + 2.0 ** -9) / (1.0 + math.exp(-(1.0 + 2.0 ** -9)))
    for dtype, ulp in (("bfloat16", 2.0 ** -8), ("float16", 2.0 ** -11)):
        out, _ = K.short_conv(x, st, w, dtype)
        got = out.item()
        assert abs(got - want) <= ulp / 2 * 1.0000001 and got != want


# tests/test_kda_prepare.py:61-123
def test_gates_hand_computed_heads():
    raw_decay = np.array([[[[0.0, 1.0], [-1.0, 2.0]]]])
    dt_bias = np.array([0.5, -0.5, 1.0, -1.0])
    a_log = np.log(np.array([2.0, 0.5])).reshape(1, 1, 2, 1)
    raw_beta = np.array([[[0.0, math.log(3.0)]]])
    q = np.array([[[3.0, 4.0, 0.0, 2.0]]])
    k = np.array([[[5.0, 12.0, 8.0, 15.0]]])
    eps = 1e-6
    decay, beta, qn, kn = K.gates(raw_decay, dt_bias, a_log, raw_beta, q, k, 2, 2, eps)
    sp = math.log1p
    want_decay = [[[[-2.0 * sp(math.exp(0.5)), -2.0 * sp(math.exp(0.5))],
                    [-0.5 * sp(math.exp(0.0)), -0.5 * sp(math.exp(1.0))]]]]
    np.testing.assert_allclose(decay, want_decay, rtol=1e-14)
    np.testing.assert_allclose(beta, [[[0.5, 0.75]]], rtol=1e-14)
    np.testing.assert_allclose(qn, [[[[3 / math.sqrt(25 + eps), 4 / math.sqrt(25 + eps)],
                                      [0.0, 2 / math.sqrt(4 + eps)]]]], rtol=1e-14)
    np.testing.assert_allclose(kn, [[[[5 / math.sqrt(169 + eps), 12 / math.sqrt(169 + eps)],
                                      [8 / math.sqrt(289 + eps), 15 / math.sqrt(289 + eps)]]]],
                               rtol=1e-14)


def test_gates_softplus_threshold_and_unit_norms():
    assert K.softplus(np.array(25.0)) == 25.0
    assert abs(K.softplus(np.array(19.9)) - math.log1p(math.exp(19.9))) < 1e-12
    assert K.softplus(np.array(-800.0)) == 0.0
    rng = np.random.default_rng(5)
    q = rng.normal(0, 3, (2, 1, 4 * 16))
    _, _, qn, kn = K.gates(np.zeros((2, 1, 4, 16)), np.zeros(64), np.zeros((1, 1, 4, 1)),
                           np.zeros((2, 1, 4)), q, q, 4, 16, 1e-30)
    np.testing.assert_allclose(np.linalg.norm(qn, axis=-1), 1.0, rtol=1e-12)


def test_planted_gate_mistakes_fail_the_hand_computed_case():
    raw_decay = np.array([[[[0.0, 1.0], [-1.0, 2.0]]]])
    dt_bias = np.array([0.5, -0.5, 1.0, -1.0])
    a_log = np.log(np.array([2.0, 0.5])).reshape(1, 1, 2, 1)
    raw_beta = np.array([[[0.0, math.log(3.0)]]])
    q = np.array([[[3.0, 4.0, 0.0, 2.0]]])
    want, _, _, _ = K.gates(raw_decay, dt_bias, a_log, raw_beta, q, q, 2, 2, 1e-6)
    # dt_bias laid out per (dim, head) instead of per (head, dim)
    swapped = dt_bias.reshape(2, 2).T.reshape(-1)
    got, _, _, _ = K.gates(raw_decay, swapped, a_log, raw_beta, q, q, 2, 2, 1e-6)
    assert not np.allclose(got, want, atol=1e-6)
