"""The group-64 packer (soc_quantize_group, host code) against the oracle's restatement of the rule, bit for bit, and
the restatement against what fixes it: the reference's per-column int8 quantizer (matrix_ops.h:42-74, itself pinned
to the compiled reference in test_oracle.py) on groups whose fp16 scale is exact, the round-trip bound, zero and
underflowing groups, and the int4 nibble layout."""
import numpy as np
import pytest

import soc_amd as S


def _rows(seed, n, k, scale=0.05):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * scale).astype(np.float16)
    w[0, :64] = 0.0                                   # zero group
    w[1, 64:128] = np.float16(1.2e-7)                 # amax / Q underflows fp16: a zero group
    w[2, :64] = np.float16(65504.0) * np.sign(rng.standard_normal(64)).astype(np.float16)  # largest values
    w[3, :64] = (np.arange(64) - 32).astype(np.float16) * np.float16(0.5)  # exact halves: round half away from zero
    return w


@pytest.mark.parametrize("bits", [8, 4])
def test_packer_equals_restatement(oracle_mod, bits):
    w = _rows(1, 37, 256)
    codes, scales = S.quantize_group(w, bits)
    rcodes, rscales = oracle_mod.quantize_group(w, bits)
    assert np.array_equal(scales, rscales)
    assert np.array_equal(codes.view(np.uint8), rcodes.view(np.uint8))


@pytest.mark.parametrize("bits", [8, 4])
def test_rule_properties(oracle_mod, bits):
    q = 127 if bits == 8 else 7
    w = _rows(2, 16, 192)
    codes, scales = oracle_mod.quantize_group(w, bits)
    deq = oracle_mod.dequant_group(codes, bits, scales, 16, 192)  # w = code * scale, exact
    s = scales.view(np.float16).astype(np.float32)
    assert s[0, 0] == 0 and s[1, 1] == 0 and np.all(deq[0, :64] == 0) and np.all(deq[1, 64:128] == 0)
    wf = w.astype(np.float32)
    if bits == 8:
        c = codes.astype(np.int32)
    else:  # unpack: even k low nibble, two's complement
        lo = (codes & 0xF).astype(np.int32)
        hi = (codes >> 4).astype(np.int32)
        c = np.empty((16, 192), np.int32)
        c[:, 0::2] = np.where(lo > 7, lo - 16, lo)
        c[:, 1::2] = np.where(hi > 7, hi - 16, hi)
    assert np.all(np.abs(c) <= q)
    sg = np.repeat(s, 64, axis=1)
    inside = (sg > 0) & (np.abs(wf) <= q * sg)
    assert np.all(np.abs(wf - c * sg)[inside] <= sg[inside] / 2 * (1 + 2 ** -20))
    # the group maximum maps to +-Q (or Q - 1 when fp16 rounding raised the scale)
    amax_code = np.max(np.abs(c).reshape(16, -1, 64), axis=2)
    assert np.all((amax_code[s > 0] >= q - 1))


def test_int8_equals_reference_per_column_rule_on_exact_scales(oracle_mod):
    """One group per column with max |w| = 127 * 2^e: the fp16 scale equals the fp32 one, so the codes must equal the
    reference quantizer's (oracle quant_int8_percol, pinned to the compiled reference)."""
    rng = np.random.default_rng(3)
    n, k = 24, 64
    e = rng.integers(-12, -2, n)
    w = (rng.uniform(-1, 1, (n, k)) * 127 * 2.0 ** e[:, None]).astype(np.float16)
    w[np.arange(n), rng.integers(0, k, n)] = (127 * 2.0 ** e).astype(np.float16)  # the exact maximum
    codes, scales = oracle_mod.quantize_group(w, 8)
    assert np.array_equal(scales.view(np.float16).astype(np.float32)[:, 0], (2.0 ** e).astype(np.float32))
    rc, rs = oracle_mod.quant_int8_percol(w.astype(np.float32).T)  # reference layout: rhs [K][N]
    assert np.array_equal(rs, (2.0 ** e).astype(np.float32))
    assert np.array_equal(codes, rc)


def test_packer_rejects_bad_shapes():
    with pytest.raises(S.SocError):
        S.quantize_group(np.zeros((2, 100), np.float16), 8)
    with pytest.raises(S.SocError):
        S.quantize_group(np.zeros((2, 64), np.float16), 5)
