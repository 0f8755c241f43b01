"""Property-based checks of the oracle (hypothesis, derandomized): invariants
that hold for every input, chosen so that a plausible slip in the restatement
-- a swapped sign, a lost term, a wrong index or shift -- fails on some
generated case. CPU only.

* codec (``mla_quant/oscar.py:130-144``): codes are monotone in the input
  within a group; a group's QDQ output takes at most four values, increasing
  with the code, from which the codes are recovered (where FP32 keeps the
  code spacing: ``|zero| <= 2^10``); negating a group maps code c to 3 - c
  away from the three thresholds (the tests are symmetric about 0: -t, 0, t);
* pack layout (this build's definition): round trip, the independent
  element-by-element packer, and one element touching only its own 2-bit field;
* window (``mla_fused_writer.py:36-51``, ``cache.py:775-800``): the rows one
  whole-sequence append keeps are exactly the read side's BF16 positions, and
  they claim distinct ring rows inside the request's own block;
* split-K (SGLang stage 2, ``rolaq_sglang.patch:94-111``): any partition of
  the keys, empty parts included, merges to the unsplit attention and LSE.
"""

import numpy as np
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st
from hypothesis.extra import numpy as hnp

from oracle import attention, codec, layout, window

PROPS = settings(max_examples=60, deadline=None, derandomize=True,
                 suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])

FINITE = st.floats(min_value=-1.0e4, max_value=1.0e4, allow_nan=False, allow_infinity=False, width=32)
GROUPS = hnp.arrays(np.float32, st.tuples(st.integers(1, 3), st.sampled_from([128, 256])), elements=FINITE)


@PROPS
@given(x=GROUPS, t=st.floats(0.5, 1.5), g=st.floats(0.8, 1.3))
def test_codec_monotone_four_levels_recoverable(x, t, g):
    codes, scale, zero, qdq = codec.lloyd_codec(torch.from_numpy(x), threshold=t, gain=g)
    rows, width = x.shape
    ng = width // 128
    xs = x.reshape(rows * ng, 128)
    cs = codes.numpy().reshape(rows * ng, 128).astype(np.int64)
    qs = qdq.numpy().reshape(rows * ng, 128)
    sc = scale.numpy().reshape(-1)
    ze = zero.numpy().reshape(-1)
    assert cs.min() >= 0 and cs.max() <= 3
    assert np.all(sc > 0) and np.all(np.isfinite(sc))
    for k in range(rows * ng):
        order = np.argsort(xs[k], kind="stable")
        assert np.all(np.diff(cs[k][order]) >= 0), "codes not monotone in the input"
        levels = {}
        for c, v in zip(cs[k], qs[k]):
            assert levels.setdefault(int(c), float(v)) == float(v), "one code, two QDQ values"
        vals = [levels[c] for c in sorted(levels)]
        assert len(vals) <= 4 and all(a < b for a, b in zip(vals, vals[1:]))
        # codes back from the QDQ values, where FP32 keeps the code spacing:
        # a group whose mean sits more than 2^10 steps from 0 (|zero| large)
        # loses it in (code - zero) * scale, in the reference as here
        if abs(float(ze[k])) <= 1024.0:
            back = np.rint(qs[k].astype(np.float64) / float(sc[k]) + float(ze[k]))
            assert np.array_equal(back.astype(np.int64), cs[k])


@PROPS
@given(x=GROUPS, t=st.floats(0.5, 1.5))
def test_codec_negation_maps_code_to_its_complement(x, t):
    c_pos = codec.lloyd_codec(torch.from_numpy(x), threshold=t)[0].numpy().astype(np.int64)
    c_neg = codec.lloyd_codec(torch.from_numpy(-x), threshold=t)[0].numpy().astype(np.int64)
    # the normalized value in float64, only to leave out elements close to a
    # threshold (where the FP32 rounding decides and the complement rule has
    # its exceptions: n == 0 gives code 2 for both signs)
    g = x.astype(np.float64).reshape(-1, 128)
    n = (g - g.mean(-1, keepdims=True)) / np.sqrt(((g - g.mean(-1, keepdims=True)) ** 2).mean(-1, keepdims=True) + 1e-8)
    n = n.reshape(x.shape)
    away = (np.abs(n) > 1e-3) & (np.abs(np.abs(n) - t) > 1e-3)
    assert np.array_equal((c_pos + c_neg)[away], np.full(int(away.sum()), 3))


@PROPS
@given(data=st.data(),
       codes=hnp.arrays(np.uint8, st.tuples(st.integers(1, 4), st.sampled_from([128, 256, 512])),
                        elements=st.integers(0, 3)))
def test_pack_roundtrip_and_field_locality(data, codes):
    rows, width = codes.shape
    packed = layout.pack_codes(codes)
    assert packed.shape == (rows, width // 4)
    assert np.array_equal(layout.unpack_codes(packed, width), codes)
    assert np.array_equal(packed, layout.pack_codes_bitwise(codes))
    r = data.draw(st.integers(0, rows - 1))
    j = data.draw(st.integers(0, width - 1))
    flipped = codes.copy()
    flipped[r, j] ^= np.uint8(data.draw(st.integers(1, 3)))
    diff = np.argwhere(layout.pack_codes(flipped) != packed)
    byte, bit = layout.element_position(j, width)
    assert diff.tolist() == [[r, int(byte)]]
    x = int(layout.pack_codes(flipped)[r, byte]) ^ int(packed[r, byte])
    assert x & ~(3 << int(bit)) == 0 and x != 0


@PROPS
@given(P=st.integers(0, 8), W=st.integers(0, 24), req=st.integers(0, 40), L=st.integers(1, 160))
def test_window_keep_equals_read_rule_and_rows_are_distinct(P, W, req, L):
    pos = np.arange(L)
    slots = np.arange(1, L + 1)
    keep = window.keep_mask(pos, np.full(L, L), np.full(L, req), slots, P, W, max_reqs=req + 1)
    assert np.array_equal(keep, window.positional_bf16(pos, L, P, W))
    rows = window.ring_row(np.full(int(keep.sum()), req), pos[keep], P, W)
    lo, hi = 1 + req * (P + W), 1 + (req + 1) * (P + W)
    assert np.all((rows >= lo) & (rows < hi))
    assert len(set(rows.tolist())) == rows.size
    # slot 0 (graph padding) and a request outside [0, max_reqs) claim nothing
    assert not window.keep_mask(pos, np.full(L, L), np.full(L, req), np.zeros(L), P, W, req + 1).any()
    assert not window.keep_mask(pos, np.full(L, L), np.full(L, req + 1), slots, P, W, req + 1).any()


@PROPS
@given(L=st.integers(1, 48), H=st.integers(1, 3), cuts=st.lists(st.integers(0, 48), max_size=6),
       empties=st.integers(0, 2), seed=st.integers(0, 2 ** 16))
def test_split_merge_over_any_partition(L, H, cuts, empties, seed):
    D, R, scale = 16, 8, 0.3
    gen = torch.Generator().manual_seed(seed)
    ql = torch.randn(1, H, D, generator=gen, dtype=torch.float64)
    qr = torch.randn(1, H, R, generator=gen, dtype=torch.float64)
    kl = 2 * torch.randn(L, D, generator=gen, dtype=torch.float64)
    kr = torch.randn(L, R, generator=gen, dtype=torch.float64)
    edges = sorted({0, L, *[min(c, L) for c in cuts]})
    bounds = list(zip(edges[:-1], edges[1:])) + [(L, L)] * empties
    parts, lses = attention.split_partials(ql, qr, kl, kr, scale, bounds)
    merged = attention.merge_splits(parts, lses)
    full, lse = attention.attend(ql, qr, kl, kr, scale, torch.float64)
    assert torch.allclose(merged, full, rtol=1e-12, atol=1e-12)
    assert torch.allclose(torch.logsumexp(lses, -1), lse, rtol=0, atol=1e-12)
