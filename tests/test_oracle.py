"""Pins the CPU oracle (oracle/lrq_oracle.c) before anything is checked
against it: reference goldens and fixture pairs, closed-form invariants,
brute-force searches and finite differences. CPU only."""

import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _golden(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def _mat(g, key):
    return np.array(g[key], dtype=np.float32)


# ---------------------------------------------------------------- int quant
@pytest.mark.parametrize("fname,qmax", [("quant_int4_golden.json", 7), ("quant_int8_golden.json", 127)])
def test_dequant_matches_reference_golden(fname, qmax):
    """tests/quant.rs:95-139: dq to 1e-6 (here value-exact), y to 1e-5."""
    g = _golden(fname)
    assert g["block"] == 32
    w, x, dq, y = (_mat(g, k) for k in ("w", "x", "dq", "y"))
    q, s = O.quantize(w, 32, qmax)
    d = O.dequant_q(q, s, 32)
    assert np.array_equal(d, dq)  # value-exact (the torch golden has -0.0 where q rounds to zero)
    yo, _ = O.linear_fwd(x, d)
    assert np.abs(yo - y).max() <= 1e-5


def test_int4_golden_through_packed_layout():
    g = _golden("quant_int4_golden.json")
    w, dq = _mat(g, "w"), _mat(g, "dq")
    q, s = O.quantize(w, 32, 7)
    packed = O.pack_int4(q)
    assert packed.shape == (8, 32)
    assert np.array_equal(O.unpack_int4(packed, 64), q)
    assert np.array_equal(O.dequant_int4(packed, s, 64, 32), dq)
    # layout: low nibble = even k, each nibble q+8
    assert (packed & 0xF).astype(int).tolist() == (q[:, 0::2].astype(int) + 8).tolist()
    assert (packed >> 4).astype(int).tolist() == (q[:, 1::2].astype(int) + 8).tolist()


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("qmax", [7, 127])
def test_roundtrip_error_bounded_by_half_a_scale_step(group, qmax):
    """tests/quant.rs:141-229 with the same ROUNDING_ULPS = 4 budget."""
    rng = np.random.Generator(np.random.PCG64(11 + group + qmax))
    w = rng.uniform(-3, 3, (16, 384)).astype(np.float32)
    q, s = O.quantize(w, group, qmax)
    d = O.dequant_q(q, s, group)
    blocks = w.reshape(16, -1, group)
    amax = np.abs(blocks).max(-1, keepdims=True)
    scale = amax / np.float32(qmax)
    budget = 4.0 * np.finfo(np.float32).eps * amax
    err = np.abs(d.reshape(blocks.shape) - blocks)
    assert (err <= scale * 0.5 + budget).all()


def test_quantize_is_the_nearest_level_brute_force():
    """Independent of the closed form: every dq is the nearest of the 15 levels
    {-7..7}*s of its block (inputs chosen away from ties)."""
    rng = np.random.Generator(np.random.PCG64(3))
    w = rng.standard_normal((12, 128)).astype(np.float32)
    q, s = O.quantize(w, 64, 7)
    for n in range(12):
        for b in range(2):
            blk = w[n, b * 64:(b + 1) * 64].astype(np.float64)
            sc = float(s[n, b])
            assert sc == np.float32(np.abs(w[n, b * 64:(b + 1) * 64]).max() / np.float32(7))
            levels = np.arange(-7, 8) * sc
            best = levels[np.abs(blk[:, None] - levels[None, :]).argmin(1)]
            assert np.array_equal(q[n, b * 64:(b + 1) * 64].astype(np.float64) * sc, best)


def test_half_away_from_zero_on_exact_ties():
    """Ties (unpinned by the reference goldens) follow Rust f32::round."""
    # block absmax 7 -> scale 1 exactly; 2.5 / -2.5 / 0.5 / -0.5 are exact ties
    blk = np.zeros((1, 32), np.float32)
    blk[0, :6] = [7.0, 2.5, -2.5, 0.5, -0.5, 6.5]
    q, s = O.quantize(blk, 32, 7)
    assert s[0, 0] == 1.0
    assert q[0, :6].tolist() == [7, 3, -3, 1, -1, 7]


def test_all_zero_block_and_bad_block():
    w = np.zeros((2, 64), np.float32)
    w[1, 40] = 1.0
    q, s = O.quantize(w, 32, 7)
    assert s.tolist() == [[0.0, 0.0], [0.0, np.float32(1.0) / np.float32(7.0)]]
    assert not q[0].any()
    with pytest.raises(ValueError, match="multiple of the quant block"):
        O.quantize(np.zeros((4, 33), np.float32), 32, 127)


def test_chunk_rows_layout_contract():
    """tests/quant.rs:330-350."""
    assert O.dequant_chunk_rows(1000, 96, 0) == [1000]
    assert O.dequant_chunk_rows(12, 96, 12 * 96 * 4) == [12]
    assert O.dequant_chunk_rows(12, 96, 96 * 4 * 5) == [4, 4, 4]
    assert O.dequant_chunk_rows(13, 96, 96 * 4 * 5) == [5, 4, 4]
    assert O.dequant_chunk_rows(4, 96, 1) == [1, 1, 1, 1]
    for d_out, d_in, b in [(53, 96, 700), (16, 96, 96 * 4 * 3), (7, 32, 200)]:
        assert sum(O.dequant_chunk_rows(d_out, d_in, b)) == d_out


def test_chunked_quantize_bit_identical_to_whole():
    """tests/quant.rs:352-395: blocks live within rows."""
    g = _golden("quant_int4_golden.json")
    w = _mat(g, "w")
    q, s = O.quantize(w, 32, 7)
    whole = O.dequant_q(q, s, 32)
    start = 0
    for rows in O.dequant_chunk_rows(8, 64, 64 * 4 * 3):
        qc, sc = O.quantize(w[start:start + rows], 32, 7)
        assert np.array_equal(O.dequant_q(qc, sc, 32), whole[start:start + rows])
        start += rows
    assert start == 8


# ---------------------------------------------------------------- fp8
def test_fp8_lut_matches_torch_golden():
    """tests/fp8.rs:608-624: bit-exact, NaN only at 0x7f/0xff."""
    lut = _golden("fp8_lut_golden.json")["lut"]
    ours = O.fp8_lut()
    for b, want in enumerate(lut):
        if want is None:
            assert np.isnan(ours[b]), hex(b)
        else:
            assert np.float32(want).view(np.uint32) == ours[b].view(np.uint32), hex(b)
    assert ours[0x7E] == 448.0 and ours[0x01] == 0.001953125


@pytest.mark.parametrize("case", ["scalar", "per_channel", "scale_shape_one"])
def test_fp8_dequant_matches_torch_golden(case):
    """tests/fp8.rs:626-662."""
    c = _golden("fp8_dequant_golden.json")[case]
    b = np.array(c["weight_bytes"], np.uint8).reshape(c["shape"])
    out = O.fp8_dequant(b, np.array(c["scale"], np.float32))
    assert np.array_equal(out.reshape(-1).view(np.uint32), np.array(c["expected"], np.float32).view(np.uint32))


def test_fp8_encoder_reproduces_reference_fixture_pairs():
    """The reference's f32 fixtures and their fp8 repacks (tiny-mmdit
    model -> model_fp8, tiny-krea2 raw -> turbo_fp8 incl. one per-channel
    tensor) pin scale = amax/448 and the RNE byte encoding exactly."""
    z = np.load(os.path.join(GOLD, "fp8_pairs.npz"))
    names = [str(n) for n in z["names"]]
    assert len(names) >= 10 and any(n.startswith("krea2_5") for n in names)
    per_channel_seen = False
    for n in names:
        key = n.split("=")[0]
        w, want_b, want_s = z[key + "_w"], z[key + "_bytes"], z[key + "_scale"]
        per_channel = want_s.size > 1
        per_channel_seen |= per_channel
        b, s = O.fp8_quantize(w, per_channel)
        assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32)), n
        assert np.array_equal(b, want_b), n
    assert per_channel_seen


def test_fp8_encode_is_nearest_even_brute_force():
    """Brute force over the decode table: nearest finite value, ties to the
    even code; saturation at +-448; sign kept on zero."""
    lut = O.fp8_lut().astype(np.float64)
    finite = np.array([b for b in range(256) if np.isfinite(lut[b])])
    rng = np.random.Generator(np.random.PCG64(5))
    vals = np.concatenate([
        rng.standard_normal(3000) * 50, rng.standard_normal(1000) * 0.01,
        lut[finite][:126] * 1.0,  # exact codes
        (lut[1:126] + lut[2:127]) / 2,  # exact midpoints (ties)
    ]).astype(np.float32)
    codes = O.fp8_encode(vals)
    for v, c in zip(vals.astype(np.float64), codes):
        if abs(v) >= 448:
            assert c & 0x7F == 0x7E
            continue
        d = np.abs(lut[finite] - v)
        best = finite[d == d.min()]
        if len(best) > 1:  # tie (same sign side): the even mantissa wins
            best = [b for b in best if (b & 1) == 0 and (np.signbit(lut[b]) == np.signbit(v) or lut[b] == 0)]
        assert abs(lut[c] - v) == d.min(), (v, c)
        if len(best) == 1:
            assert lut[c] == lut[best[0]], (v, c, best)
    assert O.fp8_encode(np.float32(-4.2e-8)) == 0x80
    assert O.fp8_encode(np.float32(500.0)) == 0x7E
    assert O.fp8_encode(np.float32(-1e9)) == 0xFE


# ---------------------------------------------------------------- linear
def test_lora_toy_golden_twenty_sgd_steps():
    """tests/lora_reference.rs:51: a fixed-constant LoraLinear trained 20 SGD
    steps (lr 0.1, MSE) reproduces torch's trained A, B and losses to 1e-5.
    Pins the oracle's LoRA forward and all three gradients together."""
    g = _golden("lora_toy.json")
    W_BASE = np.array([0.1, -0.2, 0.3, 0.4, 0.5, -0.6, -0.7, 0.8, 0.9, 0.15, -0.25, 0.35], np.float32).reshape(4, 3)
    A = np.array([0.2, 0.1, -0.3, 0.4, 0.5, -0.6, 0.7, 0.8], np.float32).reshape(4, 2)
    B = np.zeros((2, 3), np.float32)
    X = np.array([1.0, 0.5, -0.5, 0.25, -1.0, 0.3, 0.8, -0.2, 0.6, -0.7, 0.9, 0.1, 0.2, 0.4, -0.1, 1.0, -0.4,
                  0.6, 0.3, -0.8], np.float32).reshape(5, 4)
    T = np.array([0.5, -0.5, 1.0, 1.0, 0.0, -1.0, -0.3, 0.7, 0.2, 0.9, -0.1, 0.4, 0.1, 0.6, -0.6],
                 np.float32).reshape(5, 3)
    Wf = np.ascontiguousarray(W_BASE.T)  # burn [d_in, d_out] -> file layout [d_out, d_in]
    losses = []
    for _ in range(20):
        pred, _ = O.linear_fwd(X, Wf, A, B, 1.0)
        diff = pred.astype(np.float64) - T
        losses.append(float((diff ** 2).mean()))
        dY = (2.0 * diff / diff.size).astype(np.float32)
        _, dA, dB = O.linear_bwd(X, Wf, A, B, 1.0, dY)
        A = (A - np.float32(0.1) * dA).astype(np.float32)
        B = (B - np.float32(0.1) * dB).astype(np.float32)
    assert np.abs(np.array(losses) - np.array(g["losses"])).max() <= 1e-5
    assert np.abs(A.reshape(-1) - np.array(g["lora_a_final"])).max() <= 1e-5
    assert np.abs(B.reshape(-1) - np.array(g["lora_b_final"])).max() <= 1e-5


def test_backward_is_the_derivative_of_forward():
    """Finite differences of L = sum(G * Y(X, A, B)) in f64 on a tiny case."""
    rng = np.random.Generator(np.random.PCG64(9))
    M, K, N, r, s = 3, 8, 5, 2, 0.75
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((N, K)).astype(np.float32)
    A = rng.standard_normal((K, r)).astype(np.float32)
    B = rng.standard_normal((r, N)).astype(np.float32)
    G = rng.standard_normal((M, N)).astype(np.float32)
    dX, dA, dB = O.linear_bwd(X, W, A, B, s, G)

    def loss(X_, A_, B_):
        y, _ = O.linear_fwd(X_, W, A_, B_, s)
        return float((y.astype(np.float64) * G).sum())

    h = 1e-2
    for arr, grad in ((X, dX), (A, dA), (B, dB)):
        for idx in [(0, 0), (arr.shape[0] - 1, arr.shape[1] - 1), (1, 1)]:
            p = arr.copy(); p[idx] += h
            m = arr.copy(); m[idx] -= h
            args_p = [p if arr is X else X, p if arr is A else A, p if arr is B else B]
            args_m = [m if arr is X else X, m if arr is A else A, m if arr is B else B]
            fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
            assert abs(fd - grad[idx]) <= 1e-3 * max(1.0, abs(fd)), (idx, fd, grad[idx])


def test_zero_b_delta_is_a_no_op():
    """lora.rs:262-276: B = 0 makes the delta an exact no-op."""
    rng = np.random.Generator(np.random.PCG64(1))
    X = rng.standard_normal((4, 32)).astype(np.float32)
    W = rng.standard_normal((8, 32)).astype(np.float32)
    A = rng.standard_normal((32, 4)).astype(np.float32)
    y0, _ = O.linear_fwd(X, W)
    y1, _ = O.linear_fwd(X, W, A, np.zeros((4, 8), np.float32), 2.0)
    assert np.array_equal(y0, y1)


def test_cpu_baseline_step_matches_oracle():
    """The timed CPU baseline (f32 dequant + f32 GEMMs) computes the same
    fwd+bwd as the f64 oracle."""
    rng = np.random.Generator(np.random.PCG64(2))
    M, K, N, r, g = 64, 128, 96, 16, 64
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    p, s = O.quantize_int4_packed(w, g)
    X = rng.standard_normal((M, K)).astype(np.float32)
    A = rng.uniform(-0.1, 0.1, (K, r)).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 1e-2).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    st = O.CpuStepInt4(p, s, g, X, A, B, 1.0, dY)
    st.run()
    wdq = O.dequant_int4(p, s, K, g)
    assert np.array_equal(st.Wdq.view(np.uint32), wdq.view(np.uint32))  # the per-pass dequant, bit for bit
    Y, T = O.linear_fwd(X, wdq, A, B, 1.0)
    dX, dA, dB = O.linear_bwd(X, wdq, A, B, 1.0, dY)
    for got, ref in ((st.Y, Y), (st.dX, dX), (st.dA, dA), (st.dB, dB), (st.T, T)):
        assert O.rel_deviation(got, ref) < 1e-5


def test_cpu_baseline_int8_step_matches_oracle():
    """The int8 CPU baseline: its per-pass dequant is bit-identical to the
    pinned q * s (lrq_o_dequant_q, held to quant_int8_golden.json), and the
    step computes the f64 oracle's fwd+bwd."""
    rng = np.random.Generator(np.random.PCG64(4))
    M, K, N, r, g = 48, 128, 80, 8, 32
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q, s = O.quantize(w, g, 127)
    X = rng.standard_normal((M, K)).astype(np.float32)
    A = rng.uniform(-0.1, 0.1, (K, r)).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 1e-2).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    st = O.CpuStepInt8(q, s, g, X, A, B, 0.5, dY)
    st.run()
    wdq = O.dequant_q(q, s, g)
    assert np.array_equal(st.Wdq.view(np.uint32), wdq.view(np.uint32))
    Y, T = O.linear_fwd(X, wdq, A, B, 0.5)
    dX, dA, dB = O.linear_bwd(X, wdq, A, B, 0.5, dY)
    for got, ref in ((st.Y, Y), (st.dX, dX), (st.dA, dA), (st.dB, dB), (st.T, T)):
        assert O.rel_deviation(got, ref) < 1e-5


def test_cpu_baseline_forward_matches_oracle():
    """The timed few-token CPU baseline (forward only) computes the oracle's forward."""
    rng = np.random.Generator(np.random.PCG64(3))
    M, K, N, r, g = 16, 256, 200, 32, 64
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    p, s = O.quantize_int4_packed(w, g)
    X = rng.standard_normal((M, K)).astype(np.float32)
    A = rng.uniform(-0.1, 0.1, (K, r)).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 1e-2).astype(np.float32)
    st = O.CpuFwdInt4(p, s, g, X, A, B, 0.5)
    st.run()
    Y, T = O.linear_fwd(X, O.dequant_int4(p, s, K, g), A, B, 0.5)
    assert O.rel_deviation(st.Y, Y) < 1e-5 and O.rel_deviation(st.T, T) < 1e-5


def test_cpu_baseline_f32_step_matches_oracle():
    """The fp8 CPU baseline (an f32 weight decoded once, f32 GEMMs) computes
    the f64 oracle's fwd+bwd."""
    rng = np.random.Generator(np.random.PCG64(4))
    M, K, N, r = 48, 96, 64, 8
    b8, s8 = O.fp8_quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float32), True)
    W = O.fp8_dequant(b8, s8)
    X = rng.standard_normal((M, K)).astype(np.float32)
    A = rng.uniform(-0.1, 0.1, (K, r)).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 1e-2).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    st = O.CpuStepF32(W, X, A, B, 2.0, dY)
    st.run()
    Y, T = O.linear_fwd(X, W, A, B, 2.0)
    dX, dA, dB = O.linear_bwd(X, W, A, B, 2.0, dY)
    for got, ref in ((st.Y, Y), (st.dX, dX), (st.dA, dA), (st.dB, dB), (st.T, T)):
        assert O.rel_deviation(got, ref) < 1e-5
