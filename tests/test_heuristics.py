"""Pins the Session's two weight heuristics at their decision boundaries.

1. The conv "already binary" test (tbn-runtime/include/tbn/runtime/model.hpp:
   396-410): per output channel c with scale s = mean|w|, a value v is near
   when |v - (v >= 0 ? s : -s)| < 0.01*s or |v| < 0.01; the weights are
   already binary when EVERY channel has near >= 0.9 * (elements per channel).
2. The quantized Gemm's sampled check (model.hpp:765-786): the flattened B
   at i = 0, step, 2*step, ... with step = max(1, size // 1000) must be
   exactly -1, 1, 0, 0.999 or -0.999.

The expected answers come from how each input is built (how many values were
placed near, which index was spoiled), never from a restated formula, so a
changed threshold (0.9 -> 0.8), tolerance (1 % -> 10 %), an any/every slip,
a dropped |v| < 0.01 clause, a relative small-value clause, a single shared
scale, a sign-blind target or another sampling step fails one case here.

The CPU cases check the oracle (tbo_already_binary) and the test executor's
Gemm check (models.gemm_already_binary); the GPU cases feed the same weights
to the device Session, whose branch shows in its output: already-binary
conv weights give (conv(x, w >= 0) + b) * s, others conv(x, w > 0) + b; a
Gemm's already-binary B gives A @ (B >= 0), other B gives A @ (B > 0).
"""
import numpy as np
import pytest

import models
import refmath as rm

# ---------------------------------------------------------------- channel builder


def build_channel(n, s, exact, tests=(), seed=0):
    """n fp32 values whose sequential mean|v| is s up to rounding.

    `exact` values are exactly +-s (alternating signs), `tests` are placed as
    given, and the remaining far values are multiples of s from a pattern
    whose magnitudes average 1 (pairs 1.5, 0.5; a 1.75, 0.625, 0.625 triple for
    an odd count), each at least 50 % away from s and above 0.01 in
    magnitude, with alternating signs.  The first far value absorbs what the
    test values add or miss, so the mean stays s; it stays far.  Shuffled."""
    far = n - exact - len(tests)
    assert far >= 2 or (far == 0 and not tests), "builder needs two far values"
    pat = []
    if far % 2:
        pat += [1.75, 0.625, 0.625]
    pat += [1.5, 0.5] * ((far - len(pat)) // 2)
    far_mag = np.array(pat, np.float64) * s
    resid = n * s - exact * s - sum(abs(float(t)) for t in tests) - far_mag.sum()
    if far:
        far_mag[0] += resid
        assert abs(far_mag[0] - s) > 0.4 * s and far_mag[0] > 0.02
    ex = np.array([s if i % 2 == 0 else -s for i in range(exact)], np.float64)
    fv = np.array([m if i % 2 == 0 else -m for i, m in enumerate(far_mag)], np.float64)
    vals = np.concatenate([ex, np.asarray(tests, np.float64), fv]).astype(np.float32)
    np.random.default_rng(seed).shuffle(vals)
    return vals


# (name, n, exact, tests, expected) for a channel of scale s (tests in units of s
# unless absolute).  The expected answer is near-count >= 0.9 n by construction:
# `exact` values are near, each test value's nearness is stated beside it.
def channel_cases(s):
    return [
        # count threshold: ceil(0.9 n) near values pass, one fewer fails
        ("count_90_of_100", 100, 90, (), True),
        ("count_89_of_100", 100, 89, (), False),
        ("count_18_of_20", 20, 18, (), True),
        ("count_17_of_20", 20, 17, (), False),
        # tolerance 1 % of s, both signs: 0.99 % away is near, 1.01 % away is far
        ("tol_0.99pct_pos", 100, 89, (s * 1.0099,), True),
        ("tol_1.01pct_pos", 100, 89, (s * 1.0101,), False),
        ("tol_0.99pct_neg", 100, 89, (-s * 0.9901,), True),
        ("tol_1.01pct_neg", 100, 89, (-s * 0.9899,), False),
        # the absolute |v| < 0.01 clause (strict), both signs, and zeros
        ("small_0.0099", 100, 89, (0.0099,), True),
        ("small_-0.0099", 100, 89, (-0.0099,), True),
        ("small_0.0101", 100, 89, (0.0101,), False),
        ("small_0.01_exact", 100, 89, (np.float32(0.01),), False),
        ("zeros_and_neg_zero", 100, 85, (0.0, 0.0, -0.0, 0.0, -0.0), True),
        # the small-value clause is absolute: 0.02 is far even where 1 % of s is 0.04
        ("small_0.02", 100, 89, (0.02,), False),
    ]


SCALES = (1.0, 4.0, 0.5)


def _cases():
    out = []
    for s in SCALES:
        for name, n, exact, tests, want in channel_cases(s):
            if s != 4.0 and name == "small_0.02":
                continue  # with s <= 2, 1 % of s is below 0.02 anyway
            out.append(pytest.param(s, n, exact, tests, want, id=f"s{s}-{name}"))
    return out


@pytest.mark.parametrize("s,n,exact,tests,want", _cases())
def test_already_binary_single_channel(orc, s, n, exact, tests, want):
    w = build_channel(n, s, exact, tests, seed=n + exact)[None, :]
    sc = orc.channel_mean_abs(w)
    assert abs(float(sc[0]) - s) <= 1e-6 * s, "builder: mean|w| is not s"
    assert orc.already_binary(w, sc) is want


def _three_channels(bad_at, n=100):
    """Channels with scales 0.5, 3.0, 1.25: all pass (90 near) except the one
    at index bad_at (89 near)."""
    scales = (0.5, 3.0, 1.25)
    rows = [build_channel(n, s, 89 if c == bad_at else 90, (), seed=c) for c, s in enumerate(scales)]
    return np.stack(rows)


@pytest.mark.parametrize("bad_at,want", [(None, True), (0, False), (1, False), (2, False)])
def test_already_binary_every_channel(orc, bad_at, want):
    w = _three_channels(bad_at)
    assert orc.already_binary(w, orc.channel_mean_abs(w)) is want


def test_already_binary_uses_each_channels_scale(orc):
    # channel 1 holds +-3.0 exactly: near only to its own scale, not channel 0's 0.5
    w = _three_channels(None)
    sc = orc.channel_mean_abs(w)
    assert orc.already_binary(w, sc)
    assert not orc.already_binary(w, np.full(3, sc[0], np.float32))


def test_already_binary_sign_of_target(orc):
    # an all-negative channel is near -s: the target follows the value's sign
    w = -np.abs(build_channel(100, 2.0, 90, (), seed=3))[None, :]
    assert orc.already_binary(w, orc.channel_mean_abs(w))


# ---------------------------------------------------------------- Gemm sampling


def _gemm_b(size, bad_index=None, bad=0.5, fill=1.0, shape=None):
    b = np.full(size, fill, np.float32)
    b[1::2] = -fill
    if bad_index is not None:
        b[bad_index] = bad
    return b.reshape(shape) if shape else b


GEMM_CASES = [
    # step = size // 1000 = 5: samples 0, 5, ..., 4995
    ("step5_unsampled_3", 5000, 3, 0.5, True),
    ("step5_sampled_5", 5000, 5, 0.5, False),
    ("step5_last_sample_4995", 5000, 4995, 0.5, False),
    ("step5_unsampled_4999", 5000, 4999, 0.5, True),
    # below 2000 values the step is 1: every value is checked
    ("step1_size999_last", 999, 998, 0.5, False),
    ("step1_size1999_index1", 1999, 1, 0.5, False),
    ("step2_size2000_index1", 2000, 1, 0.5, True),
    ("step2_size2000_index2", 2000, 2, 0.5, False),
    # the accepted set: exact -1, 1, 0 (-0.0 equals 0), 0.999, -0.999
    ("accept_0.999", 1000, 10, 0.999, True),
    ("accept_-0.999", 1000, 10, -0.999, True),
    ("accept_zero", 1000, 10, 0.0, True),
    ("accept_neg_zero", 1000, 10, -0.0, True),
    ("reject_0.998", 1000, 10, 0.998, False),
    ("reject_-0.998", 1000, 10, -0.998, False),
    ("reject_1.0001", 1000, 10, np.float32(1.0001), False),
    ("reject_0.5", 1000, 10, 0.5, False),
    ("reject_nan", 1000, 10, np.nan, False),
]


@pytest.mark.parametrize("name,size,idx,bad,want", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_sampled_check(name, size, idx, bad, want):
    assert models.gemm_already_binary(_gemm_b(size, idx, bad)) is want


def test_gemm_sampled_check_all_accepted_values():
    vals = np.float32([-1.0, 1.0, 0.0, -0.0, 0.999, -0.999])
    assert models.gemm_already_binary(np.resize(vals, 3000))
    assert not models.gemm_already_binary(np.full(3000, 2.0, np.float32))


# ---------------------------------------------------------------- the device Session


def _conv_spec(w, b):
    M, C, kh, kw = w.shape
    H = 8
    nodes = [models.Node("conv", "Conv", ["input", "w", "b"], ["y"], {"kernel_shape": [kh, kw]})]
    y_shape = (1, M, H - kh + 1, H - kw + 1)
    return models.Spec(nodes, {"w": w, "b": b}, {"w": "float32", "b": "float32"},
                       {"input": (1, C, H, H)}, {"y": y_shape}, {"y": y_shape, "input": (1, C, H, H)})


def _run(tbn, spec, feeds):
    model = tbn.TBNModel(models.build_graph(spec, tbn))
    s = model.create_session()
    s.set_quantization(True)
    for k, v in feeds.items():
        s.set_input(k, v)
    s.run()
    return s.get_output(list(spec.outputs)[0])


def _gpu_conv_cases():
    out = []
    for name, n, exact, tests, want in channel_cases(3.0):
        if n != 100:
            continue
        out.append(pytest.param(exact, tests, want, id=name))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("exact,tests,want", _gpu_conv_cases())
def test_session_conv_heuristic(dev, tbn, orc, exact, tests, want):
    """Channel 1 (scale 3.0) carries the case; channels 0 and 2 (scales 0.5
    and 1.25) pass.  The Session must take the branch the case was built for."""
    rows = [build_channel(100, 0.5, 90, (), seed=1),
            build_channel(100, 3.0, exact, tests, seed=2),
            build_channel(100, 1.25, 90, (), seed=3)]
    w = np.stack(rows).reshape(3, 4, 5, 5)
    b = np.array([0.25, -0.5, 0.125], np.float32)
    x = np.random.default_rng(7).standard_normal((1, 4, 8, 8)).astype(np.float32)
    s = orc.channel_mean_abs(w)
    acc_ge = orc.conv2d_f64(x, np.where(w >= 0, 1.0, -1.0).astype(np.float32))
    acc_gt = orc.conv2d_f64(x, np.where(w > 0, 1.0, -1.0).astype(np.float32))
    as_binary = (acc_ge + b[None, :, None, None]) * s.astype(np.float64)[None, :, None, None]
    as_other = acc_gt + b[None, :, None, None]
    got = _run(tbn, _conv_spec(w, b), {"input": x})
    ref, other = (as_binary, as_other) if want else (as_other, as_binary)
    rm.assert_within_tolerance(got, ref, 100, np.abs(x).max() * 3.0)
    assert np.abs(got - other).max() > 0.1, "the two branches are not told apart"


def _gemm_spec(B):
    K, N = B.shape
    nodes = [models.Node("fc", "Gemm", ["a", "B"], ["y"], {})]
    return models.Spec(nodes, {"B": B}, {"B": "float32"}, {"a": (4, K)}, {"y": (4, N)},
                       {"y": (4, N), "a": (4, K)})


@pytest.mark.gpu
@pytest.mark.parametrize("name,size,idx,bad,want",
                         [c for c in GEMM_CASES if c[1] == 5000 or c[1] == 1000 and c[0] != "reject_nan"],
                         ids=[c[0] for c in GEMM_CASES if c[1] == 5000 or c[1] == 1000 and c[0] != "reject_nan"])
def test_session_gemm_heuristic(dev, tbn, name, size, idx, bad, want):
    """B[K, N] with exact zeros at sampled positions (0 and 20): the
    already-binary branch reads them as +1 (w >= 0), the other as -1 (w > 0)."""
    K = 100 if size == 5000 else 50
    B = _gemm_b(size, idx, bad)
    B[0] = 0.0
    B[20] = 0.0
    B = B.reshape(K, size // K)
    a = np.random.default_rng(11).standard_normal((4, K)).astype(np.float32)
    got = _run(tbn, _gemm_spec(B), {"a": a})
    ref_ge = a.astype(np.float64) @ np.where(B >= 0, 1.0, -1.0)
    ref_gt = a.astype(np.float64) @ np.where(B > 0, 1.0, -1.0)
    ref, other = (ref_ge, ref_gt) if want else (ref_gt, ref_ge)
    rm.assert_within_tolerance(got, ref, K, np.abs(a).max())
    assert np.abs(got - other).max() > 0.1, "the two branches are not told apart"
