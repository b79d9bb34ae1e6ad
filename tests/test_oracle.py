"""CPU: pin the oracle (oracle/convrot_oracle.c + oracle/oracle.py) before trusting it.

Each check is chosen so that a plausible mistake in the restatement -- a wrong
butterfly sign or order, a single final rounding instead of per-op rounding,
round-half-away instead of half-even, a transposed repack, a dropped epilogue
term -- fails at least one of them:

* known answers from /root/reference/tests/test_core.py (literal pack bytes
  :186-192, repack shape :203-211, radix transform vs kron :177-184);
* closed forms (the regular Hadamard sign formula; exact integer dots);
* an independent arithmetic restatement of the eager graph in torch bf16/f16
  (torch rounds every elementwise op to the tensor dtype, RNE -- the MLX eager
  semantics the reference's oracle runs with);
* brute force on tiny inputs and hand-computed quantization cases;
* sensitivity checks: deliberately wrong variants built on the CPU must differ.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)


def kron_hadamard(size: int) -> np.ndarray:
    """test_core.py:42-50."""
    m = H4
    while m.shape[0] < size:
        m = np.kron(m, H4)
    return m / np.sqrt(size)


def sign_formula_hadamard(size: int) -> np.ndarray:
    """H[i][j] = (-1)^{#base-4 digits d with i_d + j_d = 3} / sqrt(G)."""
    s = int(round(math.log(size, 4)))
    h = np.empty((size, size))
    for i in range(size):
        for j in range(size):
            n = sum(1 for d in range(s) if ((i >> (2 * d)) & 3) + ((j >> (2 * d)) & 3) == 3)
            h[i, j] = (-1) ** n
    return h / np.sqrt(size)


TORCH_DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def torch_from(orc, bits, dtype):
    return torch.from_numpy(orc.to_f32(bits, dtype)).to(TORCH_DT[dtype])


def torch_eager_hadamard(x: torch.Tensor, group_size: int) -> torch.Tensor:
    """core.py:79-94 in torch ops on the input dtype (every op rounds to it)."""
    features = x.shape[-1]
    groups = features // group_size
    prefix = (*x.shape[:-1], groups)
    y = x.reshape(*prefix, group_size)
    stride = 1
    while stride < group_size:
        y = y.reshape(*prefix, group_size // (4 * stride), 4, stride)
        a, b, c, d = y[..., 0, :], y[..., 1, :], y[..., 2, :], y[..., 3, :]
        y = torch.stack([a + b + c - d, a + b - c + d, a - b + c + d, -a + b + c + d], dim=-2)
        y = y.reshape(*prefix, group_size)
        stride *= 4
    return (y / math.sqrt(group_size)).reshape(x.shape)


def torch_eager_quantize(x: torch.Tensor):
    """core.py:154-158 in torch ops on the input dtype."""
    absmax = x.abs().amax(dim=-1, keepdim=True)
    absmax = torch.maximum(absmax, torch.tensor(1e-10, dtype=x.dtype))
    scales = absmax / 7
    q = torch.clamp(torch.round(x / scales), -7, 7).to(torch.int8)  # torch.round: half to even
    return q, scales.reshape(-1).to(torch.float32)


# ------------------------------------------------------------------ dtype conversions


def test_bf16_conversion_matches_torch(orc):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x00000001, 0x3F808000,
                         0x3F818000, 0x3F80FFFF, 0x477FE000], dtype=np.uint32)
    f = np.concatenate([bits, specials]).view(np.float32)
    finite = np.isfinite(f)
    ours = orc.from_f32(f[finite], "bfloat16")
    ref = torch.from_numpy(f[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_conversion_matches_numpy(orc):
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.normal(0, 1, 1 << 18), rng.normal(0, 1e-5, 1 << 18), rng.normal(0, 3e4, 1 << 16),
                        np.array([65504.0, 65520.0, 65519.99, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                                  6.1e-5, 0.0, -0.0])]).astype(np.float32)
    ours = orc.from_f32(f, "float16")
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16)
    assert np.array_equal(ours, ref.view(np.uint16))
    assert np.array_equal(orc.to_f32(ours, "float16"), ref.astype(np.float32))


# ------------------------------------------------------------------ rotation


@pytest.mark.parametrize("G", [4, 16, 64, 256])
def test_sign_formula_equals_kron(G):
    assert np.array_equal(sign_formula_hadamard(G), kron_hadamard(G))


@pytest.mark.parametrize("G", [64, 256])
def test_radix_transform_matches_regular_hadamard_fp32(orc, G):
    """test_core.py:177-184: float32 rotation vs x @ H within 2e-6."""
    rng = np.random.default_rng(17)
    values = rng.normal(size=(3, 512)).astype(np.float32)
    result = orc.regular_hadamard(values, "float32", G)
    h = kron_hadamard(G)
    expected = np.concatenate([values[:, i:i + G] @ h for i in range(0, 512, G)], axis=1)
    np.testing.assert_allclose(result, expected, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("seed,shape,G", [(1802, (19, 512), 256), (2026082305, (17, 2688), 64),
                                          (17, (19, 512), 16), (5, (7, 1024), 4), (6, (5, 2048), 1024)])
def test_rotation_matches_torch_eager(orc, dtype, seed, shape, G):
    """Per-op rounding: the C restatement equals the eager graph evaluated by torch."""
    rng = np.random.default_rng(seed)
    x = orc.from_f32(rng.normal(size=shape).astype(np.float32), dtype)
    ours = orc.to_f32(orc.regular_hadamard(x, dtype, G), dtype)
    ref = torch_eager_hadamard(torch_from(orc, x, dtype), G).to(torch.float32).numpy()
    assert np.array_equal(ours, ref)


def test_rotation_single_rounding_would_differ(orc):
    """Sensitivity: rotating in float32 and rounding once gives different values."""
    rng = np.random.default_rng(20260823)
    x = orc.from_f32(rng.normal(size=(64, 3072)).astype(np.float32), "bfloat16")
    ours = orc.regular_hadamard(x, "bfloat16", 256)
    xf = orc.to_f32(x, "bfloat16").astype(np.float64)
    h = kron_hadamard(256)
    once = np.concatenate([xf[:, i:i + 256] @ h for i in range(0, 3072, 256)], axis=1).astype(np.float32)
    assert (orc.from_f32(once, "bfloat16") != ours).mean() > 0.01


# ------------------------------------------------------------------ quantization


def test_pack_layout_literal_bytes(orc):
    """test_core.py:186-192."""
    values = np.array([[-8, -7, -1, 0, 1, 7, 3, -4]], dtype=np.int8)
    packed = orc.pack_signed_int4(values)
    assert packed.tolist() == [[0x98, 0x0F, 0x71, 0xC3]]
    assert orc.unpack_signed_int4(packed).tolist() == values.tolist()


def test_quantize_hand_computed_ties(orc):
    """absmax 7 -> scale 1: ratios are exact, rint is half-to-even (2.5 -> 2, 3.5 -> 4)."""
    row = np.array([[7, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, 0]], dtype=np.float32)
    codes, scales = orc.quantize_rowwise_codes(orc.from_f32(row, "bfloat16"), "bfloat16")
    assert codes.tolist() == [[7, 2, 4, -2, -4, 0, 2, 0]]
    assert scales.tolist() == [1.0]


def test_quantize_zero_row_and_floor(orc):
    row = np.zeros((1, 16), np.float32)
    codes, scales = orc.quantize_rowwise_codes(orc.from_f32(row, "bfloat16"), "bfloat16")
    assert not codes.any()
    floor = orc.to_f32(orc.from_f32(np.array([1e-10], np.float32), "bfloat16"), "bfloat16")[0]
    expected = orc.to_f32(orc.from_f32(np.array([floor / 7], np.float32), "bfloat16"), "bfloat16")[0]
    assert scales[0] == expected


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("seed,shape", [(23, (19, 256)), (28, (19, 1024)), (1801, (64, 512))])
def test_quantize_matches_torch_eager(orc, dtype, seed, shape):
    rng = np.random.default_rng(seed)
    x = orc.from_f32(rng.normal(size=shape).astype(np.float32), dtype)
    codes, scales = orc.quantize_rowwise_codes(x, dtype)
    q, s = torch_eager_quantize(torch_from(orc, x, dtype))
    assert np.array_equal(codes, q.numpy())
    assert np.array_equal(scales, s.numpy())


@pytest.mark.parametrize("seed", [18, 1801, 20260823])
def test_prepare_matches_torch_eager_and_invariants(orc, seed):
    """prepare = quantize(rotate(x)) (core.py:161-167) on the reference seeds."""
    rng = np.random.default_rng(seed)
    x = orc.from_f32(rng.normal(size=(19, 512)).astype(np.float32), "bfloat16")
    codes, scales = orc.prepare_codes(x, "bfloat16", 256)
    q, s = torch_eager_quantize(torch_eager_hadamard(torch_from(orc, x, "bfloat16"), 256))
    assert np.array_equal(codes, q.numpy()) and np.array_equal(scales, s.numpy())
    assert codes.min() >= -7 and codes.max() <= 7  # -8 is never emitted
    assert (np.abs(codes).max(axis=1) == 7).all()
    assert np.array_equal(orc.to_f32(orc.from_f32(scales, "bfloat16"), "bfloat16"), scales)


def test_quantize_round_half_away_would_differ(orc):
    """Sensitivity: rounding ties away from zero changes codes of real rows."""
    rng = np.random.default_rng(20260823)
    x = orc.from_f32(rng.normal(size=(256, 3072)).astype(np.float32), "bfloat16")
    r = orc.to_f32(orc.regular_hadamard(x, "bfloat16", 256), "bfloat16")
    codes, scales = orc.quantize_rowwise_codes(orc.from_f32(r, "bfloat16"), "bfloat16")
    ratio = orc.to_f32(orc.from_f32(r / scales[:, None], "bfloat16"), "bfloat16")
    away = np.clip(np.sign(ratio) * np.floor(np.abs(ratio) + 0.5), -7, 7)
    assert (away != codes).sum() > 0


def test_reciprocal_multiply_is_exact_for_bf16():
    """The HIP prep kernel divides by the scale as x * rcp(scale).  For bf16 operands
    RN_bf16(RN_f32(x * r')) == RN_bf16(x / s) for every reciprocal r' within 1 ulp of
    RN_f32(1/s): checked exhaustively over all 128 x 128 bf16 significand pairs and both
    relative exponents that reach the code range."""
    sig = np.arange(128, dtype=np.float64)
    xs = (1.0 + sig / 128.0)
    ss = (1.0 + sig / 128.0)

    def rn_bf16(v):
        return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()

    bad = 0
    for e in (-3, -2, -1, 0, 1, 2):
        x = (xs * 2.0 ** e)[:, None]
        s = ss[None, :]
        exact = rn_bf16((x / s).astype(np.float64))  # RN of the exact quotient (double is exact enough)
        rcp = (1.0 / s.astype(np.float32)).astype(np.float32)
        for ulp in (-1, 0, 1):
            r = np.nextafter(rcp, np.float32(np.inf if ulp > 0 else -np.inf)) if ulp else rcp
            prod = (x.astype(np.float32) * r).astype(np.float32)
            bad += int((rn_bf16(prod) != exact).sum())
    assert bad == 0


# ------------------------------------------------------------------ layouts


def test_mpp_repack_shape_and_round_trip(orc):
    """test_core.py:203-211."""
    rng = np.random.default_rng(2026082301)
    v = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    nk = orc.pack_signed_int4(v)
    kn = orc.repack_nk_weight_for_mpp(nk)
    assert kn.shape == (64, 23)
    assert np.array_equal(orc.repack_mpp_weight_to_nk(kn), nk)


def test_mpp_repack_brute_force(orc):
    rng = np.random.default_rng(3)
    v = rng.integers(-8, 8, size=(6, 10), dtype=np.int8)
    kn = orc.repack_nk_weight_for_mpp(orc.pack_signed_int4(v))
    for n in range(6):
        for k in range(10):
            nib = (int(kn[k, n // 2]) >> (4 * (n % 2))) & 0xF
            assert (nib - 16 if nib >= 8 else nib) == v[n, k]


def test_cdna4_layout_brute_force(orc):
    """Every (n, k) lands at block [k//128][n//16], byte 16*(16q + n%16) + 4c + j with
    k%128 = 32q + 8c + 4h + j, low nibble for h=0 -- the layout the GEMMs read."""
    rng = np.random.default_rng(4)
    N, K = 37, 300
    v = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    blocks = orc.codes_to_cdna4(v)
    assert blocks.shape == (3, 3, 1024)
    for n in range(N):
        for k in range(K):
            kk = k % 128
            q, c, h, j = kk // 32, (kk // 8) % 4, (kk // 4) % 2, kk % 4
            byte = int(blocks[k // 128, n // 16, 16 * (16 * q + n % 16) + 4 * c + j])
            nib = (byte >> (4 * h)) & 0xF
            assert (nib - 16 if nib >= 8 else nib) == v[n, k]
    pad = orc.cdna4_to_codes(blocks, 48, 384)
    assert not pad[N:].any() and not pad[:, K:].any()
    assert np.array_equal(orc.cdna4_to_codes(blocks, N, K), v)


def test_fp6_codes_are_the_integers_over_8(orc):
    """The FP6 fields of -8 .. 7, decoded by the e2m3 definition (bias 1, 3 mantissa bits),
    are the codes divided by 8: no two share a field, 0 has no sign bit, |v| <= 7 are
    subnormals (exponent bits zero, mantissa |v|), and a scan of all 64 fields finds
    exactly these among the fields whose value times 8 is an integer of [-8, 7] (0 aside)."""
    v = np.arange(-8, 8)
    c = orc.fp6_code(v)
    assert np.array_equal(orc.e2m3_value(c) * 8.0, v.astype(np.float64))
    assert np.array_equal(orc.fp6_value(c), v.astype(np.float64))
    assert len(set(c.tolist())) == 16 and int(c[8]) == 0
    small = np.abs(v) <= 7
    assert not ((c[small] >> 3) & 3).any() and np.array_equal(c[small] & 7, np.abs(v[small]))
    assert int(c[0]) == 0b101000  # -8/8 = -1.0: sign, exponent 1 (bias 1), mantissa 0
    all_codes = np.arange(64)
    vals = orc.e2m3_value(all_codes) * 8.0
    ints = {int(x): int(k) for k, x in zip(all_codes, vals)
            if x == np.round(x) and -8 <= x <= 7 and not (x == 0 and k)}
    assert ints == {int(x): int(k) for x, k in zip(v, c)}
    for bad in (-9, 8):
        with pytest.raises(ValueError):
            orc.fp6_code(np.array([bad]))


def test_bf16_ratios_stay_below_7_5(orc):
    """Every bf16 ratio is at most 7.03125 in magnitude, so rint(ratio) never leaves [-7, 7]
    and the clamp (core.py:157) never binds: for every positive finite bf16 row maximum m,
    scale = bf16(max(m, bf16(1e-10)) / 7), and the largest ratio bf16(m * RN(1/scale)) and
    bf16(m / scale) (the division the reference runs) are at most 7.03125."""
    bits = np.arange(0x0001, 0x7F80, dtype=np.uint32)  # positive finite bf16 (subnormals included)
    m = (bits << 16).view(np.float32)
    floor = orc.to_f32(orc.from_f32(np.array([1e-10], np.float32), "bfloat16"), "bfloat16")[0]
    scale = orc.to_f32(orc.from_f32((np.maximum(m, floor) / np.float32(7)).astype(np.float32), "bfloat16"),
                       "bfloat16")
    inv = (np.float32(1) / scale).astype(np.float32)
    by_rcp = orc.to_f32(orc.from_f32((m * inv).astype(np.float32), "bfloat16"), "bfloat16")
    by_div = orc.to_f32(orc.from_f32((m / scale).astype(np.float32), "bfloat16"), "bfloat16")
    assert by_rcp.max() <= 7.03125 and by_div.max() <= 7.03125
    assert by_rcp.max() > 7.0  # the bound is reached, not loose


def test_fp6_zero_code_sign_fix_over_all_bf16_pairs():
    """The preparation kernel's zero_code_sign_fix (prep.hip), restated on every bf16 half:
    h & ~((h + 0x40ff mod 2^16) & 0x8000) clears the sign of exactly the negative values of
    magnitude <= 0.5 (whose code rint(x) is 0) and leaves every other value unchanged."""
    h = np.arange(65536, dtype=np.uint32)
    fixed = h & ~(((h + 0x40FF) & 0xFFFF) & 0x8000)
    x = (h << 16).view(np.float32)
    finite = np.isfinite(x)
    zero_code = finite & (np.abs(x) <= 0.5)
    assert np.array_equal(fixed[zero_code], h[zero_code] & 0x7FFF)
    assert np.array_equal(fixed[~zero_code & finite], h[~zero_code & finite])
    assert np.array_equal(np.rint(x[zero_code]), np.zeros(int(zero_code.sum())))  # code 0 indeed
    assert not np.any(np.rint(np.abs(x[finite & ~zero_code])) == 0)


def test_fp6_layout_brute_force(orc):
    """Every (r, k) lands in block [k//128][r//16], lane L = 16*(k%128//32) + r%16, as the
    6 bits at 6*(k%32) of the lane's 24-byte stream (bytes 0..15 at 16*L, 16..23 at
    1024 + 8*L), built bit by bit here; the lanes hold the same features as the CDNA4
    layout's lanes."""
    rng = np.random.default_rng(6)
    R, K = 37, 256
    v = rng.integers(-8, 8, size=(R, K), dtype=np.int8)
    blocks = orc.codes_to_fp6(v)
    assert blocks.shape == (2, 3, 1536)
    want = np.zeros_like(blocks)
    for r in range(R):
        for k in range(K):
            kb, kk = divmod(k, 128)
            L = 16 * (kk // 32) + r % 16
            code = int(orc.fp6_code(np.array([v[r, k]]))[0])
            for b in range(6):
                bit = 6 * (kk % 32) + b
                byte = 16 * L + bit // 8 if bit < 128 else 1024 + 8 * L + (bit - 128) // 8
                want[kb, r // 16, byte] |= ((code >> b) & 1) << (bit % 8)
    assert np.array_equal(blocks, want)
    assert np.array_equal(orc.fp6_to_codes(blocks, R, K), v)
    cd = orc.cdna4_to_codes(orc.codes_to_cdna4(v), R, K)
    assert np.array_equal(cd, v)  # same (row, feature) -> lane assignment: lane 16*(k%128//32) + r%16


def test_fp6c_masks_are_the_exponent_bits(orc):
    """The compact layout's masks, derived from the e2m3 field layout: field i of a lane's
    16-field run sits at stream bits 6i .. 6i+5 with its exponent at 6i+3, 6i+4; Z0 / Z1 are
    those positions inside dwords D0 / D1, and D2's exponent positions are exactly the bits in
    neither mask (so D2's information bits fill D0's and D1's exponent bits)."""
    exp_bits = [6 * i + b for i in range(16) for b in (3, 4)]
    masks = [sum(1 << (p - 32 * d) for p in exp_bits if 32 * d <= p < 32 * d + 32) for d in range(3)]
    assert masks[0] == orc.FP6C_Z0 and masks[1] == orc.FP6C_Z1
    assert orc.FP6C_Z0 & orc.FP6C_Z1 == 0
    assert orc.FP6C_Z0 | orc.FP6C_Z1 == ~masks[2] & 0xFFFFFFFF
    assert bin(orc.FP6C_Z0).count("1") + bin(orc.FP6C_Z1).count("1") + bin(masks[2]).count("1") == 32


def test_fp6c_layout_round_trips_every_code_at_every_position(orc):
    """Every code -7 .. 7 at every one of a lane's 32 positions (the rest random), in a ragged
    37 x 256 operand: expanding the compact blocks gives the FP6 operand blocks bit for bit,
    and the codes come back.  Swapping the masks (a plausible slip) does not round-trip."""
    rng = np.random.default_rng(66)
    R, K = 37, 256
    for v in range(-7, 8):
        c = rng.integers(-7, 8, size=(R, K), dtype=np.int8)
        c[:, (np.arange(K) + v) % 32 == 0] = v
        c[np.arange(R) % 5 == 0] = v
        blocks = orc.codes_to_fp6c(c)
        assert blocks.shape == (2, 3, 1024)
        assert np.array_equal(orc.fp6c_expand(blocks), orc.codes_to_fp6(c))
        assert np.array_equal(orc.fp6c_to_codes(blocks, R, K), c)
    i = np.ascontiguousarray(blocks).view("<u4").reshape(2, 3, 64, 4)
    z0, z1 = np.uint32(orc.FP6C_Z1), np.uint32(orc.FP6C_Z0)  # swapped
    d2 = (i[..., 0] & z0) | (i[..., 1] & z1)
    want = orc.codes_to_fp6(c)[..., :1024].view("<u4").reshape(2, 3, 64, 4)[..., 2]
    assert not np.array_equal(d2, want)
    with pytest.raises(ValueError, match="-7 .. 7"):
        orc.codes_to_fp6c(np.full((16, 128), -8, np.int8))


# ------------------------------------------------------------------ matmuls


def test_w4a4_integer_dots_exact(orc):
    """test_core.py:244-264: unit scales and zero bias give the exact integer dot."""
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-8, 8, size=(37, 64), dtype=np.int8)
    w = rng.integers(-8, 8, size=(46, 64), dtype=np.int8)
    out, dots = orc.w4a4_matmul_codes(a, w, np.ones(37, np.float32), np.ones(46, np.float32),
                                      np.zeros(46, np.float32), "float32", want_dots=True)
    exact = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(dots, exact) and np.array_equal(out, exact.astype(np.float32))


def test_w4a4_epilogue_order(orc):
    """((dot * xs) * ws) + bias as separate float32 ops (core.py:1168-1170): equal to numpy
    float32 arithmetic in that order, and within 1e-6 of the float64 value (test_core.py:240)."""
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-7, 8, size=(37, 64), dtype=np.int8)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(37,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    out = orc.w4a4_matmul_codes(a, w, xs, ws, b, "float32")
    dots = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    np32 = ((dots * xs[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32) + b[None, :]
    assert np.array_equal(out, np32)
    f64 = dots.astype(np.float64) * xs[:, None] * ws[None, :] + b[None, :]
    np.testing.assert_allclose(out, f64, rtol=1e-6, atol=1e-6)
    fused = (dots.astype(np.float64) * xs[:, None] * ws[None, :] + b[None, :]).astype(np.float32)
    assert not np.array_equal(out, np.float32(0) + dots * xs[:, None]), "a dropped term must change the output"
    assert np.abs(out - fused).max() < 1e-5


@pytest.mark.parametrize("out_dtype", ["float32", "bfloat16", "float16"])
def test_w4a4_large_path_equals_int64_path(orc, out_dtype):
    """The full-size checker (float32 BLAS dots + C epilogue) equals the int64 oracle bit for
    bit, including extreme codes (-8 everywhere at K = 15360: |dot| = 64 K, the largest the
    float32 argument allows) and a ragged slab boundary."""
    rng = np.random.default_rng(29)
    a = rng.integers(-8, 8, size=(67, 2688), dtype=np.int8)
    w = rng.integers(-8, 8, size=(53, 2688), dtype=np.int8)
    xs = rng.uniform(0.001, 0.2, size=(67,)).astype(np.float32)
    ws = rng.uniform(0.001, 0.2, size=(53,)).astype(np.float32)
    b = rng.normal(size=(53,)).astype(np.float32)
    want = orc.w4a4_matmul_codes(a, w, xs, ws, b, out_dtype)
    got = orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype)
    assert np.array_equal(got.view(np.uint32) if out_dtype == "float32" else got,
                          want.view(np.uint32) if out_dtype == "float32" else want)
    K = 15360
    a8 = np.full((3, K), -8, np.int8)
    w8 = np.full((2, K), -8, np.int8)
    w8[1, ::2] = 7
    dots = orc.w4a4_dots_exact(a8, w8)
    assert np.array_equal(dots, a8.astype(np.int64) @ w8.astype(np.int64).T)
    # a dropped term (one code zeroed) must show in the dots
    a8[0, 5] = 0
    assert orc.w4a4_dots_exact(a8, w8)[0, 0] == 64 * K - 64


def test_w4a4_bf16_output_is_rounded_float32(orc):
    rng = np.random.default_rng(27)
    a = rng.integers(-7, 8, size=(31, 1024), dtype=np.int8)
    w = rng.integers(-7, 8, size=(61, 1024), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(31,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(61,)).astype(np.float32)
    b = rng.normal(size=(61,)).astype(np.float32)
    f32 = orc.w4a4_matmul_codes(a, w, xs, ws, b, "float32")
    bf = orc.w4a4_matmul_codes(a, w, xs, ws, b, "bfloat16")
    assert np.array_equal(bf, orc.from_f32(f32, "bfloat16"))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_w4a16_matches_float64(orc, dtype):
    """test_core.py:285-309 tolerance: rtol 1e-6, atol 1e-5 against (act @ codes.T) * ws + b."""
    rng = np.random.default_rng(2026082303)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    act = orc.from_f32(rng.normal(size=(37, 64)).astype(np.float32), dtype)
    out, dots, mag = orc.w4a16_matmul_codes(act, dtype, w, ws, b, "float32")
    af = orc.to_f32(act, dtype).astype(np.float64)
    ref = (af @ w.astype(np.float64).T) * ws[None, :] + b[None, :]
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-5)
    assert np.allclose(mag, np.abs(af) @ np.abs(w.astype(np.float64)).T, rtol=1e-6)
