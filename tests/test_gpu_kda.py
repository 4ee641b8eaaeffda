"""GPU parity of the KDA decode kernels (local_kimi_amd/csrc/kda.hip) with oracle/kda.py.

Tolerances, stated per test: the recurrence step within 3e-5 absolute +
3e-5 relative of the float64 oracle after one step at the real shape and
5e-4 after 256 chained steps (the reference's own bounds,
tests/test_kda_step.py:9-12); the short convolutions within one unit in the
last place of a 16-bit storage dtype (four for fp32) plus the fp32 error of
the four-term sum (the oracle rounds the exact value, the kernel its fp32
sum) and the shifted states bit-exact; the gates within 1e-5
relative + 1e-6 absolute (fp32 arithmetic against float64). Reruns are
bit-identical, and a captured graph replays bit-identically to eager calls.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda as K

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd import _lib

    _lib.load()


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def _np(t):
    return t.detach().double().cpu().numpy()


def _step_inputs(rng, b, h, dk, dv, state_std=0.05):
    state = state_std * rng.normal(size=(b, h, dk, dv))
    q = rng.normal(size=(b, h, dk))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = rng.normal(size=(b, h, dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = 0.2 * rng.normal(size=(b, h, dv))
    decay = -(0.005 + 0.075 * rng.uniform(size=(b, h, dk)))
    beta = 1.0 / (1.0 + np.exp(-rng.normal(size=(b, h))))
    return [a.astype(np.float32) for a in (state, q, k, v, decay, beta)]


def _close(actual, expected, atol, rtol, what):
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    worst = float((err / bound).max())
    assert worst <= 1.0, f"{what}: worst error {worst:.3f} of the bound (max abs {err.max():.3g})"


# ---------------------------------------------------------------------------
# recurrence step


@pytest.mark.parametrize("b,h,dk,dv", [(1, 32, 128, 128), (2, 3, 64, 96), (1, 2, 200, 40),
                                       (3, 1, 16, 30), (1, 1, 128, 1)])
def test_step_matches_oracle(rng, b, h, dk, dv):
    from local_kimi_amd.kernels import kda_decode_step

    state, q, k, v, decay, beta = _step_inputs(rng, b, h, dk, dv)
    scale = dk ** -0.5
    want_state, want_out = K.decode_step(state, q, k, v, decay, beta, scale)
    st = _t(state)
    out = kda_decode_step(st, _t(q), _t(k), _t(v), _t(decay), _t(beta), scale=scale)
    _close(_np(st), want_state, 3e-5, 3e-5, f"state {b, h, dk, dv}")
    _close(_np(out), want_out, 3e-5, 3e-5, f"output {b, h, dk, dv}")
    # a rerun from the same state is bit-identical
    st2 = _t(state)
    out2 = kda_decode_step(st2, _t(q), _t(k), _t(v), _t(decay), _t(beta), scale=scale)
    assert torch.equal(st, st2) and torch.equal(out, out2)


def test_step_error_stays_bounded_after_256_steps(rng):
    """256 chained steps from a zero state (4 heads of 128 x 128)."""
    from local_kimi_amd.kernels import kda_decode_step

    steps, b, h, d = 256, 1, 4, 128
    want = np.zeros((b, h, d, d))
    st = torch.zeros((b, h, d, d), dtype=torch.float32, device=DEV)
    for _ in range(steps):
        _, q, k, v, decay, beta = _step_inputs(rng, b, h, d, d)
        want, want_out = K.decode_step(want, q, k, v, decay, beta, d ** -0.5)
        out = kda_decode_step(st, _t(q), _t(k), _t(v), _t(decay), _t(beta), scale=d ** -0.5)
    _close(_np(st), want, 5e-4, 5e-4, "state after 256 steps")
    _close(_np(out), want_out, 5e-4, 5e-4, "output after 256 steps")


def test_step_updates_a_strided_state_in_place(rng):
    from local_kimi_amd.kernels import kda_decode_step

    state, q, k, v, decay, beta = _step_inputs(rng, 1, 2, 32, 32)
    want_state, want_out = K.decode_step(state, q, k, v, decay, beta, 0.25)
    big = torch.zeros((1, 2, 32, 64), dtype=torch.float32, device=DEV)
    view = big[..., :32]
    view.copy_(_t(state))
    out = kda_decode_step(view, _t(q), _t(k), _t(v), _t(decay), _t(beta), scale=0.25)
    _close(_np(big[..., :32]), want_state, 3e-5, 3e-5, "strided state")
    _close(_np(out), want_out, 3e-5, 3e-5, "strided state output")
    assert torch.count_nonzero(big[..., 32:]) == 0


def test_step_rejects_wide_keys():
    from local_kimi_amd.kernels import kda_decode_step

    st = torch.zeros((1, 1, 257, 8), device=DEV)
    z = torch.zeros((1, 1, 257), device=DEV)
    with pytest.raises(ValueError, match="d_k up to 256"):
        kda_decode_step(st, z, z, torch.zeros((1, 1, 8), device=DEV), z,
                        torch.zeros((1, 1), device=DEV), scale=1.0)


# ---------------------------------------------------------------------------
# short convolutions

_STORAGE = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _ulp(values: np.ndarray, dtype) -> np.ndarray:
    mant = {torch.float32: 23, torch.float16: 10, torch.bfloat16: 7}[dtype]
    tiny = {torch.float32: 2.0 ** -126, torch.float16: 2.0 ** -14, torch.bfloat16: 2.0 ** -126}[dtype]
    mag = np.maximum(np.abs(values), tiny)
    return 2.0 ** (np.floor(np.log2(mag)) - mant)


def _conv_bound(want, x, st, w, dtype):
    """One unit in the last place of a 16-bit storage dtype (the same value
    rounded on either side of a boundary), four for fp32 storage (expf, the
    divide and the final rounding of SiLU in fp32), plus the fp32 accumulation
    error of a four-term sum, 4 * 2^-24 of the sum of the products'
    magnitudes (SiLU's slope stays under 1.1)."""
    w = np.asarray(w, np.float64).reshape(-1, 4)
    window = np.concatenate((np.asarray(st)[:, :, 1:], np.asarray(x)[:, 0, :, None]), axis=-1)
    mag = (np.abs(window) * np.abs(w)[None]).sum(axis=-1)[:, None, :]
    ulps = 4.0 if dtype == torch.float32 else 1.0
    return ulps * _ulp(want, dtype) * 1.000001 + 1.1 * 4 * 2.0 ** -24 * mag


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,c", [(2, 4096), (1, 300), (3, 1)])
def test_short_conv_matches_oracle(rng, dtype, b, c):
    from local_kimi_amd.kernels import fused_short_conv_triple

    name = _STORAGE[dtype]
    vals = [K.round_to(rng.normal(size=(b, 1, c)), name) for _ in range(3)]
    states = [K.round_to(rng.normal(size=(b, c, 4)), name) for _ in range(3)]
    weights = [K.round_to(0.5 * rng.normal(size=(c, 1, 4)), name) for _ in range(3)]
    outs_want, states_want = K.short_conv_triple(*vals, *states, *weights, name)
    dev_states = [_t(s, dtype) for s in states]
    outs = fused_short_conv_triple(*(_t(v, dtype) for v in vals), *dev_states,
                                   *(_t(w, dtype) for w in weights))
    for o, want, x, st, w in zip(outs, outs_want, vals, states, weights):
        assert o.dtype == dtype and tuple(o.shape) == (b, 1, c)
        err = np.abs(_np(o) - want)
        assert (err <= _conv_bound(want, x, st, w, dtype)).all(), f"{name}: {err.max():.3g}"
    for s, want in zip(dev_states, states_want):
        assert np.array_equal(_np(s), want)


def test_short_conv_weights_in_another_dtype_and_strided_state(rng):
    from local_kimi_amd.kernels import fused_short_conv_triple

    b, c = 2, 64
    vals = [K.round_to(rng.normal(size=(b, 1, c)), "bfloat16") for _ in range(3)]
    states = [K.round_to(rng.normal(size=(b, c, 4)), "bfloat16") for _ in range(3)]
    weights = [rng.normal(size=(c, 4)).astype(np.float32) for _ in range(3)]
    outs_want, states_want = K.short_conv_triple(*vals, *states, *weights, "bfloat16")
    bounds = [_conv_bound(o, x, st, w, torch.bfloat16)
              for o, x, st, w in zip(outs_want, vals, states, weights)]
    bigs = [torch.zeros((b, c, 8), dtype=torch.bfloat16, device=DEV) for _ in range(3)]
    views = [big[..., 2:6] for big in bigs]
    for v, s in zip(views, states):
        v.copy_(_t(s, torch.bfloat16))
    outs = fused_short_conv_triple(*(_t(v, torch.bfloat16) for v in vals), *views,
                                   *(_t(w) for w in weights))
    for o, want, bound in zip(outs, outs_want, bounds):
        assert (np.abs(_np(o) - want) <= bound).all()
    for big, want in zip(bigs, states_want):
        assert np.array_equal(_np(big[..., 2:6]), want)
        assert torch.count_nonzero(big[..., :2]) == 0 and torch.count_nonzero(big[..., 6:]) == 0


# ---------------------------------------------------------------------------
# gates


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,s,h,d,flat", [(2, 1, 32, 128, True), (1, 3, 4, 72, False),
                                          (1, 1, 2, 1000, True)])
def test_gates_match_oracle(rng, dtype, b, s, h, d, flat):
    from local_kimi_amd.kernels import fused_kda_gates

    name = _STORAGE[dtype]
    raw_decay = K.round_to(2.0 * rng.normal(size=(b, s, h, d)), name)
    raw_decay.reshape(-1)[:3] = [25.0, 19.5, -30.0]  # both sides of the softplus threshold
    dt_bias = rng.normal(size=h * d).astype(np.float32)
    a_log = np.log(rng.uniform(1.0, 16.0, size=h)).astype(np.float32).reshape(1, 1, h, 1)
    raw_beta = K.round_to(rng.normal(size=(b, s, h)), name)
    shape = (b, s, h * d) if flat else (b, s, h, d)
    q = K.round_to(rng.normal(size=shape), name)
    k = K.round_to(3.0 * rng.normal(size=shape), name)
    want = K.gates(raw_decay, dt_bias, a_log, raw_beta, q, k, h, d, 1e-6)
    got = fused_kda_gates(_t(raw_decay, dtype), _t(dt_bias), _t(a_log), _t(raw_beta, dtype),
                          _t(q, dtype), _t(k, dtype), num_heads=h, head_dim=d, eps=1e-6)
    for g, w, what in zip(got, want, ("decay", "beta", "q", "k")):
        assert g.dtype == torch.float32 and tuple(g.shape) == w.shape, what
        _close(_np(g), w, 1e-6, 1e-5, what)


# ---------------------------------------------------------------------------
# the decode chain under graph replay


def test_prepare_and_step_graph_replays_match_eager(rng):
    """Convolutions, gates and the step for one layer (B=1, 32 heads of 128,
    bf16 projections), captured once; four replays against the same chain run
    eagerly on copies of the states, bit for bit, with eager work between."""
    from local_kimi_amd.kernels import fused_kda_gates, fused_short_conv_triple, kda_decode_step

    h, d = 32, 128
    c = h * d
    bf = torch.bfloat16
    ins = [_t(K.round_to(rng.normal(size=(1, 1, c)), "bfloat16"), bf) for _ in range(3)]
    conv_w = [_t(K.round_to(0.3 * rng.normal(size=(c, 1, 4)), "bfloat16"), bf) for _ in range(3)]
    raw_decay = _t(K.round_to(rng.normal(size=(1, 1, h, d)), "bfloat16"), bf)
    raw_beta = _t(K.round_to(rng.normal(size=(1, 1, h)), "bfloat16"), bf)
    dt_bias = _t(rng.normal(size=c).astype(np.float32))
    a_log = _t(np.log(rng.uniform(1, 16, size=h)).astype(np.float32).reshape(1, 1, h, 1))

    def chain(conv_states, rec):
        q, k, v = fused_short_conv_triple(*ins, *conv_states, *conv_w)
        decay, beta, qn, kn = fused_kda_gates(raw_decay, dt_bias, a_log, raw_beta, q, k,
                                              num_heads=h, head_dim=d, eps=1e-6)
        vv = v.view(1, 1, h, d).float()
        return kda_decode_step(rec, qn[:, 0], kn[:, 0], vv[:, 0], decay[:, 0], beta[:, 0],
                               scale=d ** -0.5)

    conv0 = [torch.zeros((1, c, 4), dtype=bf, device=DEV) for _ in range(3)]
    rec0 = 0.05 * torch.randn((1, h, d, d), device=DEV)
    g_conv = [t.clone() for t in conv0]
    g_rec = rec0.clone()
    e_conv = [t.clone() for t in conv0]
    e_rec = rec0.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        chain([t.clone() for t in conv0], rec0.clone())  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        g_out = chain(g_conv, g_rec)
    for rep in range(4):
        with torch.cuda.stream(stream):
            graph.replay()
        e_out = chain(e_conv, e_rec)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out), rep
        assert torch.equal(g_rec, e_rec), rep
        for a, b in zip(g_conv, e_conv):
            assert torch.equal(a, b), rep
        _ = (e_rec.sum() * 2).item()  # unrelated eager work between replays


# ---------------------------------------------------------------------------
# the whole layer in one launch


def _layer_inputs(rng, b, h, d, name):
    c = h * d
    ins = [K.round_to(rng.normal(size=(b, 1, c)), name) for _ in range(3)]
    conv_states = [K.round_to(rng.normal(size=(b, c, 4)), name) for _ in range(3)]
    conv_w = [K.round_to(0.3 * rng.normal(size=(c, 1, 4)), name) for _ in range(3)]
    raw_decay = K.round_to(rng.normal(size=(b, 1, h, d)), name)
    raw_beta = K.round_to(rng.normal(size=(b, 1, h)), name)
    dt_bias = rng.normal(size=c).astype(np.float32)
    a_log = np.log(rng.uniform(1, 16, size=h)).astype(np.float32).reshape(1, 1, h, 1)
    rec = (0.05 * rng.normal(size=(b, h, d, d))).astype(np.float32)
    return ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec


@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, None), (torch.float16, None),
                                           (torch.float32, None), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("b,h,d", [(1, 32, 128), (2, 4, 72), (3, 2, 8)])
def test_layer_matches_the_oracle_chain(rng, dtype, wdtype, b, h, d):
    """Convolutions (states bit-exact), gates and step against the oracle's
    composition, within the step's single-step bound (3e-5). Covers fp32
    values (conv outputs not rounded) and fp32 conv weights with bf16 values."""
    from local_kimi_amd.kernels import kda_decode_layer

    name = _STORAGE[dtype]
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, name)
    # weights of another dtype keep their bf16 values (stored as fp32), so the
    # conv products stay exact and the bf16-rounded outputs stay comparable
    wdtype = wdtype or dtype
    (qo, ko, vo), states_want = K.short_conv_triple(*ins, *conv_states, *conv_w, name)
    decay, beta, qn, kn = K.gates(raw_decay, dt_bias, a_log, raw_beta, qo, ko, h, d, 1e-6)
    want_state, want_out = K.decode_step(rec, qn[:, 0], kn[:, 0], vo.reshape(b, h, d),
                                         decay[:, 0], beta[:, 0], d ** -0.5)
    dev_states = [_t(s, dtype) for s in conv_states]
    st = _t(rec)
    out = kda_decode_layer(*(_t(x, dtype) for x in ins), *dev_states,
                           *(_t(w, wdtype) for w in conv_w), _t(raw_decay, dtype), _t(dt_bias),
                           _t(a_log), _t(raw_beta, dtype), st, num_heads=h, head_dim=d)
    for s, want in zip(dev_states, states_want):
        assert np.array_equal(_np(s), want)
    _close(_np(st), want_state, 3e-5, 3e-5, f"layer state {b, h, d}")
    _close(_np(out), want_out, 3e-5, 3e-5, f"layer output {b, h, d}")


def test_layer_agrees_with_the_three_launch_chain(rng):
    """Same inputs through fused_short_conv_triple + fused_kda_gates +
    kda_decode_step: conv states bit-identical, state and output within the
    rounding of two summation orders (1e-6 absolute + 1e-5 relative)."""
    from local_kimi_amd.kernels import (fused_kda_gates, fused_short_conv_triple,
                                        kda_decode_layer, kda_decode_step)

    b, h, d = 2, 32, 128
    bf = torch.bfloat16
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, "bfloat16")
    args = [_t(x, bf) for x in ins], [_t(w, bf) for w in conv_w]
    s1 = [_t(s, bf) for s in conv_states]
    s2 = [_t(s, bf) for s in conv_states]
    r1, r2 = _t(rec), _t(rec)
    out1 = kda_decode_layer(*args[0], *s1, *args[1], _t(raw_decay, bf), _t(dt_bias), _t(a_log),
                            _t(raw_beta, bf), r1, num_heads=h, head_dim=d)
    q, k, v = fused_short_conv_triple(*args[0], *s2, *args[1])
    decay, beta, qn, kn = fused_kda_gates(_t(raw_decay, bf), _t(dt_bias), _t(a_log),
                                          _t(raw_beta, bf), q, k, num_heads=h, head_dim=d,
                                          eps=1e-6)
    out2 = kda_decode_step(r2, qn[:, 0], kn[:, 0], v.view(b, h, d).float(), decay[:, 0],
                           beta[:, 0], scale=d ** -0.5)
    for a, c in zip(s1, s2):
        assert torch.equal(a, c)
    _close(_np(r1), _np(r2), 1e-6, 1e-5, "layer vs chain state")
    _close(_np(out1), _np(out2), 1e-6, 1e-5, "layer vs chain output")


def test_layer_graph_replays_match_eager(rng):
    from local_kimi_amd.kernels import kda_decode_layer

    b, h, d = 1, 32, 128
    bf = torch.bfloat16
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, "bfloat16")
    fixed = ([_t(x, bf) for x in ins], [_t(w, bf) for w in conv_w], _t(raw_decay, bf),
             _t(dt_bias), _t(a_log), _t(raw_beta, bf))

    def run(states, r):
        return kda_decode_layer(*fixed[0], *states, *fixed[1], fixed[2], fixed[3], fixed[4],
                                fixed[5], r, num_heads=h, head_dim=d)

    g_states, e_states = [_t(s, bf) for s in conv_states], [_t(s, bf) for s in conv_states]
    g_rec, e_rec = _t(rec), _t(rec)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run([_t(s, bf) for s in conv_states], _t(rec))
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        g_out = run(g_states, g_rec)
    for rep in range(4):
        with torch.cuda.stream(stream):
            graph.replay()
        e_out = run(e_states, e_rec)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out) and torch.equal(g_rec, e_rec), rep
        for a, c in zip(g_states, e_states):
            assert torch.equal(a, c), rep


def test_layer_rejects_wide_heads():
    from local_kimi_amd.kernels import kda_decode_layer

    h, d = 1, 132
    c = h * d
    bf = torch.bfloat16
    x = torch.zeros((1, 1, c), dtype=bf, device=DEV)
    s = torch.zeros((1, c, 4), dtype=bf, device=DEV)
    w = torch.zeros((c, 1, 4), dtype=bf, device=DEV)
    with pytest.raises(ValueError, match="multiple of 4 up to 128"):
        kda_decode_layer(x, x, x, s, s.clone(), s.clone(), w, w, w,
                         torch.zeros((1, 1, h, d), dtype=bf, device=DEV),
                         torch.zeros(c, device=DEV), torch.zeros((1, 1, h, 1), device=DEV),
                         torch.zeros((1, 1, h), dtype=bf, device=DEV),
                         torch.zeros((1, h, d, d), device=DEV), num_heads=h, head_dim=d)


# ---------------------------------------------------------------------------
# the layer over several blocks per head (conv states double-buffered)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b,h,d", [(1, 32, 128), (2, 4, 72), (3, 2, 8), (1, 3, 64)])
def test_split_layer_matches_the_oracle_chain(rng, dtype, b, h, d):
    """New conv states (written to the other buffer) bit-exact, the old ones
    untouched, state and output within the step's single-step bound (3e-5).
    (2, 4, 72): 5 column blocks per head, the last one half empty; (1, 3, 64):
    an item count that is no multiple of 16 (blocks in plain order)."""
    from local_kimi_amd.kernels import kda_decode_layer

    name = _STORAGE[dtype]
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, name)
    (qo, ko, vo), states_want = K.short_conv_triple(*ins, *conv_states, *conv_w, name)
    decay, beta, qn, kn = K.gates(raw_decay, dt_bias, a_log, raw_beta, qo, ko, h, d, 1e-6)
    want_state, want_out = K.decode_step(rec, qn[:, 0], kn[:, 0], vo.reshape(b, h, d),
                                         decay[:, 0], beta[:, 0], d ** -0.5)
    old = [_t(s, dtype) for s in conv_states]
    new = [torch.full_like(s, 7.0) for s in old]
    st = _t(rec)
    out = kda_decode_layer(*(_t(x, dtype) for x in ins), *old, *(_t(w, dtype) for w in conv_w),
                           _t(raw_decay, dtype), _t(dt_bias), _t(a_log), _t(raw_beta, dtype), st,
                           num_heads=h, head_dim=d, conv_states_out=new)
    for s, want, before in zip(new, states_want, conv_states):
        assert np.array_equal(_np(s), want)
    for s, before in zip(old, conv_states):
        assert np.array_equal(_np(s), before)
    _close(_np(st), want_state, 3e-5, 3e-5, f"split layer state {b, h, d}")
    _close(_np(out), want_out, 3e-5, 3e-5, f"split layer output {b, h, d}")


def test_split_layer_tokens_agree_with_the_one_block_layer(rng):
    """Four decode tokens, the split layer alternating two conv-state sets and
    the one-block layer updating its states in place: conv states equal after
    every token; state and output within two summation orders (1e-6 absolute
    + 1e-5 relative per token)."""
    from local_kimi_amd.kernels import kda_decode_layer

    b, h, d = 2, 32, 128
    bf = torch.bfloat16
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, "bfloat16")
    fixed = ([_t(w, bf) for w in conv_w], _t(raw_decay, bf), _t(dt_bias), _t(a_log),
             _t(raw_beta, bf))
    one = [_t(s, bf) for s in conv_states]
    sets = [[_t(s, bf) for s in conv_states], [torch.zeros_like(_t(s, bf)) for s in conv_states]]
    r_one, r_split = _t(rec), _t(rec)
    for token in range(4):
        x = [_t(K.round_to(rng.normal(size=(b, 1, h * d)), "bfloat16"), bf) for _ in range(3)]
        o1 = kda_decode_layer(*x, *one, *fixed[0], *fixed[1:], r_one, num_heads=h, head_dim=d)
        src, dst = sets[token % 2], sets[(token + 1) % 2]
        o2 = kda_decode_layer(*x, *src, *fixed[0], *fixed[1:], r_split, num_heads=h, head_dim=d,
                              conv_states_out=dst)
        for a, c in zip(one, dst):
            assert torch.equal(a, c), token
        _close(_np(r_split), _np(r_one), 1e-6, 1e-5, f"token {token} state")
        _close(_np(o2), _np(o1), 1e-6, 1e-5, f"token {token} output")
        r_split.copy_(r_one)  # the next token starts both layers from the same state


def test_split_layer_graph_replays_match_eager(rng):
    from local_kimi_amd.kernels import kda_decode_layer

    b, h, d = 1, 32, 128
    bf = torch.bfloat16
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, "bfloat16")
    fixed = ([_t(x, bf) for x in ins], [_t(w, bf) for w in conv_w], _t(raw_decay, bf),
             _t(dt_bias), _t(a_log), _t(raw_beta, bf))
    src = [_t(s, bf) for s in conv_states]

    def run(dst, r):
        return kda_decode_layer(*fixed[0], *src, *fixed[1], *fixed[2:], r, num_heads=h,
                                head_dim=d, conv_states_out=dst)

    g_dst, e_dst = [torch.zeros_like(s) for s in src], [torch.zeros_like(s) for s in src]
    g_rec, e_rec = _t(rec), _t(rec)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run([torch.zeros_like(s) for s in src], _t(rec))
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        g_out = run(g_dst, g_rec)
    for rep in range(4):
        with torch.cuda.stream(stream):
            graph.replay()
        e_out = run(e_dst, e_rec)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out) and torch.equal(g_rec, e_rec), rep
        for a, c in zip(g_dst, e_dst):
            assert torch.equal(a, c), rep


def test_split_layer_refuses_outputs_that_overlap_the_states(rng):
    from local_kimi_amd.kernels import kda_decode_layer

    b, h, d = 1, 2, 8
    bf = torch.bfloat16
    ins, conv_states, conv_w, raw_decay, raw_beta, dt_bias, a_log, rec = _layer_inputs(
        rng, b, h, d, "bfloat16")
    states = [_t(s, bf) for s in conv_states]
    args = ([_t(x, bf) for x in ins], [_t(w, bf) for w in conv_w])
    with pytest.raises(ValueError, match="overlaps"):
        kda_decode_layer(*args[0], *states, *args[1], _t(raw_decay, bf), _t(dt_bias), _t(a_log),
                         _t(raw_beta, bf), _t(rec), num_heads=h, head_dim=d,
                         conv_states_out=(states[0], torch.zeros_like(states[1]),
                                          torch.zeros_like(states[2])))
