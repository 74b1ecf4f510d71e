"""Pins for the oracle functions that no reference golden vector covers: the
K-quant weight quantizers (ggml quantize_row_q{4,5,6}_K_ref, called through
ggml_quantize_chunk at tools/quantize/quantize_rows.cpp:210), the Q8_K
activation rounding rule, and the ggml-cuda right-operand formats Q8_1 and
Q8_1-D4 (tools/validation/verify_q8_rhs_staging.py:24-83,
tools/quantize/native_activation.py:42-62).

Each check states a property the mathematics of the published algorithm fixes
and is evaluated independently of the oracle's arithmetic (float64 least
squares, exhaustive candidate sets, nearest-grid searches, exact grids), so a
slipped constant, a missing candidate, a wrong weight or a wrong sign fails:
  * the sub-block fit is the best of ggml's published candidate search, no
    better and no worse (Q4_K: 21 inverse scales (14 + 0.1 i)/(max - min)
    plus the plain one, weights sqrt(mean x^2) + |x|; Q5_K: 16 from 30.5;
    Q6_K: 19 symmetric scales -(32 + 0.1 i)/max, weights x^2);
  * the 6-bit (Q4_K/Q5_K) and 8-bit (Q6_K) scale codes are the nearest codes
    of the fitted scales with the largest one at 63 / -128, and d, dmin are
    the fp16 values of max/63 and -max/128;
  * every final code is a nearest point of its sub-block's decoded grid;
  * sub-blocks lying on an exact grid come back with exactly that grid;
  * Q8_K rounds ties to even, and its sign convention cancels in every dot.
CPU only."""

import json
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))

F32 = np.float32
ASYM = {12: (15, -1.0, 20), 13: (31, -0.5, 15)}      # type -> (nmax, rmin, nstep)


def _f16(v):
    return float(np.float16(np.float32(v)))


def _unpack_scale_min(b12):
    """6-bit scale/min j of a Q4_K/Q5_K header: j<4 low 6 bits of bytes j,
    j+4; j>=4 a nibble of byte j+4 and the top two bits of bytes j-4 / j."""
    b = [int(v) for v in b12]
    sc, mn = [], []
    for j in range(8):
        if j < 4:
            sc.append(b[j] & 63)
            mn.append(b[j + 4] & 63)
        else:
            sc.append((b[j + 4] & 15) | ((b[j - 4] >> 6) << 4))
            mn.append((b[j + 4] >> 4) | ((b[j] >> 6) << 4))
    return np.array(sc), np.array(mn)


def _asym_codes(qtype, blk):
    """256 codes of a Q4_K / Q5_K super-block (layout pinned by the
    field-by-field packer in test_oracle.py)."""
    qs = blk[16:144] if qtype == 12 else blk[48:176]
    codes = np.zeros(256, np.int64)
    for e in range(256):
        j, l = e // 32, e % 32
        v = (int(qs[32 * (j // 2) + l]) >> (4 * (j % 2))) & 15
        if qtype == 13:
            v |= ((int(blk[16 + l]) >> j) & 1) << 4
        codes[e] = v
    return codes


def _q6_codes(blk):
    codes = np.zeros(256, np.int64)
    for e in range(256):
        half, r = e // 128, e % 128
        quarter, l = r // 32, r % 32
        lo = (int(blk[64 * half + 32 * (quarter % 2) + l]) >> (4 * (quarter // 2))) & 15
        hi = (int(blk[128 + 32 * half + l]) >> (2 * quarter)) & 3
        codes[e] = lo | (hi << 4)
    return codes


def _superblocks(seed, count):
    """Super-blocks of varied character: N(0, 0.02^2) weights, heavy tails,
    one-signed blocks, outliers and mixed sub-block magnitudes."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        kind = i % 6
        if kind == 0:
            x = rng.standard_normal(256) * 0.02
        elif kind == 1:
            x = rng.standard_t(2, 256) * 0.01
        elif kind == 2:
            x = np.abs(rng.standard_normal(256)) * 0.03 + 0.001
        elif kind == 3:
            x = -np.abs(rng.standard_normal(256)) * 0.03
        elif kind == 4:
            x = rng.standard_normal(256) * 0.02
            x[rng.integers(0, 256, 3)] *= 40
        else:
            x = rng.standard_normal(256) * (10.0 ** rng.uniform(-4, 0, 256)) * 0.1
        out.append(x.astype(np.float32))
    return out


# ---- the sub-block fits against the published candidate search -----------

def _asym_search(x, w, nmax, rmin, nstep):
    """ggml's make_qkx2_quants search on one sub-block, evaluated in float64
    except for the codes (float32 products rounded to nearest even, as the
    published nearest_int does): the plain inverse scale nmax/(max - min),
    then (rmin + 0.1 i + nmax)/(max - min) for i = 0..nstep, each candidate's
    codes refitted by weighted least squares (min <= 0) and kept when its
    error is lower; a kept candidate's min replaces `min` for the later
    candidates.  Returns (codes, scale, -min, error)."""
    lo = min(F32(x.min()), F32(0))
    hi = F32(x.max())
    xd = x.astype(np.float64)
    iscale = F32(nmax) / (hi - lo)
    L = np.clip(np.rint(iscale * (x - lo)), 0, nmax).astype(np.float64)
    scale, mn = 1.0 / float(iscale), float(lo)
    best = float((w * (scale * L + mn - xd) ** 2).sum())
    for i in range(nstep + 1):
        iscale = (F32(rmin) + F32(0.1) * F32(i) + F32(nmax)) / (hi - lo)
        Lc = np.clip(np.rint(iscale * (x - lo)), 0, nmax).astype(np.float64)
        sw, sl, sl2, sx, sxl = w.sum(), (w * Lc).sum(), (w * Lc * Lc).sum(), (w * xd).sum(), (w * Lc * xd).sum()
        det = sw * sl2 - sl * sl
        if det <= 0:
            continue
        a = (sw * sxl - sx * sl) / det
        b = (sl2 * sx - sl * sxl) / det
        if b > 0:
            b, a = 0.0, sxl / sl2
        err = float((w * (a * Lc + b - xd) ** 2).sum())
        if err < best:
            L, scale, mn, best, lo = Lc, a, b, err, F32(b)
    return L, scale, -mn, best


@pytest.mark.parametrize("qtype", [12, 13])
def test_asym_fit_follows_the_published_search(oracle, qtype):
    """The oracle's fit against an independent float64 evaluation of the
    published search: the same codes in at least 99 % of the sub-blocks, and
    there the same least-squares scale and min."""
    nmax, rmin, nstep = ASYM[qtype]
    total = same = 0
    for x256 in _superblocks(11 + qtype, 300):
        scales, mins, codes = oracle.kquant_fit(qtype, x256)
        for j in range(8):
            x = x256[32 * j:32 * j + 32]
            xd = x.astype(np.float64)
            w = np.sqrt((xd * xd).mean()) + np.abs(xd)
            if x.max() == min(x.min(), 0):
                assert scales[j] == 0 and (codes[32 * j:32 * j + 32] == 0).all()
                continue
            L = codes[32 * j:32 * j + 32].astype(np.float64)
            assert L.max() <= nmax
            tL, tscale, tmin, terr = _asym_search(x, w, nmax, rmin, nstep)
            err = float((w * (float(scales[j]) * L - float(mins[j]) - xd) ** 2).sum())
            floor = 1e-12 * float((w * xd * xd).sum())
            total += 1
            if np.array_equal(L, tL):
                same += 1
                assert abs(float(scales[j]) - tscale) <= 1e-3 * abs(tscale)
                assert abs(float(mins[j]) - tmin) <= 1e-3 * abs(tscale) * nmax
                assert err <= terr * (1 + 1e-6) + floor, (qtype, j, err, terr)
    # float32 near-ties send a few searches down another path (0.25 % of
    # sub-blocks here); a wrong candidate set or weight moves far more
    assert same >= 0.99 * total, (same, total)


def _sym_metric(x, L):
    w = x.astype(np.float64) ** 2
    sl2 = (w * L * L).sum()
    return ((w * x * L).sum() ** 2 / sl2) if sl2 > 0 else 0.0


def test_q6_fit_is_the_best_published_candidate(oracle):
    nmax = 32
    for x256 in _superblocks(7, 300):
        scales, _, codes = oracle.kquant_fit(14, x256)
        for s in range(16):
            x = x256[16 * s:16 * s + 16]
            amax_i = int(np.argmax(np.abs(x)))
            if np.abs(x).max() < 1e-15:
                assert scales[s] == 0
                continue
            mx = F32(x[amax_i])
            L = codes[16 * s:16 * s + 16].astype(np.int64) - nmax
            assert L.min() >= -nmax and L.max() <= nmax - 1
            cands = []
            for i in [0] + [i for i in range(-9, 10) if i != 0]:
                iscale = -(F32(nmax) + F32(0.1) * F32(i)) / mx if i else F32(-nmax) / mx
                Lc = np.clip(np.rint(iscale * x), -nmax, nmax - 1).astype(np.float64)
                cands.append(_sym_metric(x, Lc))
            got = _sym_metric(x, L.astype(np.float64))
            best = max(cands)
            assert got >= best * (1 - 1e-5) and got <= best * (1 + 1e-5), (s, got, best)
            w = x.astype(np.float64) ** 2
            ls = (w * x * L).sum() / (w * L * L).sum()
            assert abs(float(scales[s]) - ls) <= 1e-5 * abs(ls)


# ---- scale codes and super-block scales -----------------------------------

@pytest.mark.parametrize("qtype", [12, 13])
def test_asym_scale_codes_and_header(oracle, qtype):
    for x256 in _superblocks(21 + qtype, 200):
        scales, mins, _ = oracle.kquant_fit(qtype, x256)
        blk = oracle.quantize(qtype, x256.reshape(1, 256))[0]
        d = float(blk[0:2].view(np.float16)[0])
        dmin = float(blk[2:4].view(np.float16)[0])
        sc, mn = _unpack_scale_min(blk[4:16])
        for vals, codes, scale in ((scales, sc, d), (mins, mn, dmin)):
            top = float(vals.max())
            if top <= 0:
                assert scale == 0 and (codes == 0).all()
                continue
            assert scale == _f16(F32(top) / F32(63))           # d = fp16(max / 63)
            assert codes[int(np.argmax(vals))] == 63          # the largest one stores 63
            ideal = 63.0 * vals.astype(np.float64) / top
            assert (np.abs(codes - ideal) <= 0.5 + 1e-4).all()  # nearest 6-bit code of each


def test_q6_scale_codes_and_header(oracle):
    for x256 in _superblocks(31, 200):
        scales, _, _ = oracle.kquant_fit(14, x256)
        blk = oracle.quantize(14, x256.reshape(1, 256))[0]
        if np.abs(scales).max() < 1e-15:
            assert (blk == 0).all()
            continue
        sc = blk[192:208].view(np.int8).astype(np.int64)
        d = float(blk[208:210].view(np.float16)[0])
        top = float(scales[int(np.argmax(np.abs(scales)))])
        for s in np.flatnonzero(np.abs(scales) == np.abs(scales).max()):
            assert sc[s] == -128                                # largest |scale| stores -128
        assert abs(d - (-top / 128.0)) <= float(np.spacing(np.float16(abs(d))))
        ideal = np.minimum(-128.0 * scales.astype(np.float64) / top, 127.49)
        assert (np.abs(sc - ideal) <= 0.5 + 1e-4).all()


# ---- final codes: nearest grid point ----------------------------------------

@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_final_codes_are_nearest_grid_points(oracle, qtype):
    for x256 in _superblocks(41 + qtype, 120):
        blk = oracle.quantize(qtype, x256.reshape(1, 256))[0]
        y = oracle.dequantize(qtype, blk.reshape(1, -1), 256)[0].astype(np.float64)
        if qtype == 14:
            d = F32(blk[208:210].view(np.float16)[0])
            sc = blk[192:208].view(np.int8)
            for s in range(16):
                ds = F32(d * F32(sc[s]))
                if ds == 0:
                    continue
                grid = (ds * np.arange(-32, 32, dtype=np.float32)).astype(np.float64)
                x = x256[16 * s:16 * s + 16].astype(np.float64)
                nearest = np.abs(x[:, None] - grid[None, :]).min(axis=1)
                assert (np.abs(x - y[16 * s:16 * s + 16]) <= nearest + 1e-6 * abs(float(ds))).all()
        else:
            nmax = ASYM[qtype][0]
            d = F32(blk[0:2].view(np.float16)[0])
            dmin = F32(blk[2:4].view(np.float16)[0])
            sc, mn = _unpack_scale_min(blk[4:16])
            for j in range(8):
                dj, mj = F32(d * F32(sc[j])), F32(dmin * F32(mn[j]))
                if dj == 0:
                    continue
                grid = (dj * np.arange(nmax + 1, dtype=np.float32) - mj).astype(np.float64)
                x = x256[32 * j:32 * j + 32].astype(np.float64)
                nearest = np.abs(x[:, None] - grid[None, :]).min(axis=1)
                assert (np.abs(x - y[32 * j:32 * j + 32]) <= nearest + 1e-6 * abs(float(dj))).all()


# ---- exact grids and zero blocks ------------------------------------------------

@pytest.mark.parametrize("qtype,shift", [(12, 0.0), (12, 0.05), (13, 0.0), (13, 0.07)])
def test_asym_exact_grid_round_trip(oracle, qtype, shift):
    nmax = ASYM[qtype][0]
    rng = np.random.default_rng(qtype)
    q = np.concatenate([rng.permutation(np.resize(np.arange(nmax + 1), 32)) for _ in range(8)])
    x = (F32(0.01) * q.astype(np.float32) - F32(shift)).astype(np.float32)
    blk = oracle.quantize(qtype, x.reshape(1, 256))[0]
    sc, mn = _unpack_scale_min(blk[4:16])
    assert (sc == 63).all() and ((mn == 63).all() if shift else (mn == 0).all())
    assert np.array_equal(_asym_codes(qtype, blk), q)


def test_q6_exact_grid_round_trip(oracle):
    rng = np.random.default_rng(6)
    q = np.concatenate([np.concatenate([[-32], rng.integers(-31, 32, 15)]) for _ in range(16)])
    x = (F32(0.003) * q.astype(np.float32)).astype(np.float32)
    blk = oracle.quantize(14, x.reshape(1, 256))[0]
    assert (blk[192:208].view(np.int8) == -128).all()
    assert np.array_equal(_q6_codes(blk) - 32, q)


@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_zero_superblock_packs_to_zeros(oracle, qtype):
    blk = oracle.quantize(qtype, np.zeros((2, 256), np.float32))
    assert not blk.any()


def test_scale_min_unpack_inverts_the_field_packer():
    from tests.test_oracle import _pack_scale_min_bits
    rng = np.random.default_rng(5)
    for _ in range(50):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        got_sc, got_mn = _unpack_scale_min(_pack_scale_min_bits(sc, mn))
        assert np.array_equal(got_sc, sc) and np.array_equal(got_mn, mn)


# ---- Q8_K rounding and sign ---------------------------------------------------

@pytest.mark.parametrize("lead", [-127.0, 127.0])
def test_q8_k_ties_round_to_even(oracle, lead):
    # |iscale| = 127/127 = 1 exactly, so iscale * x is exactly +-0.5, 1.5, ...
    x = np.zeros((1, 256), np.float32)
    x[0, :8] = [lead, 0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5]
    blk = oracle.quantize(oracle.Q8_K, x)[0]
    d = blk[0:4].view(np.float32)[0]
    q = blk[4:12].view(np.int8).astype(np.int64)
    sign = -1 if lead > 0 else 1                        # iscale = -127 / (signed maximum)
    assert d == sign * 1.0
    # ties to even (0.5 -> 0, 2.5 -> 2, -2.5 -> -2), not away from zero
    assert (q * sign).tolist() == [int(lead), 0, 2, 2, 4, 0, -2, -2]
    assert (d * q.astype(np.float32)).tolist() == np.rint(x[0, :8]).tolist()


def test_q8_k_sign_convention_cancels_in_every_dot(oracle):
    # Negating the stored scale and codes of every Q8_K block leaves each
    # K-quant dot bit-identical, so the product path does not depend on it.
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    for qtype in (12, 13, 14):
        w = oracle.quantize(qtype, (rng.standard_normal((5, 512)) * 0.02).astype(np.float32))
        xq = oracle.quantize(oracle.Q8_K, x)
        flipped = xq.copy().reshape(3, 2, 292)
        flipped[:, :, 0:4] = (-flipped[:, :, 0:4].copy().view(np.float32)).view(np.uint8)
        flipped[:, :, 4:260] = (-flipped[:, :, 4:260].view(np.int8)).view(np.uint8)
        flipped[:, :, 260:292] = (-flipped[:, :, 260:292].copy().view(np.int16)).view(np.uint8)
        flipped = flipped.reshape(3, -1)
        for n in range(5):
            for m in range(3):
                a = oracle.lib().or_vec_dot(qtype, w[n].ctypes.data, xq[m].ctypes.data, 512)
                b = oracle.lib().or_vec_dot(qtype, w[n].ctypes.data, flipped[m].ctypes.data, 512)
                assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


# ---- ggml-cuda Q8_1 and Q8_1-D4 ---------------------------------------------------

def _q8_1_rules(values, payload):
    """The reference verifier's acceptance rules for Q8_1 blocks
    (tools/validation/verify_q8_rhs_staging.py:24-83): the fp16 scale is the
    nearest of amax/127 (or its neighbour at a tie within 4 F32 ulps), codes
    round half away from zero (adjacent only at such ties), the stored sum is
    the fp16 of the 32-lane xor-butterfly F32 sum of the original values."""
    values = np.asarray(values, np.float32).reshape(-1, 32)
    payload = np.asarray(payload, np.uint8).reshape(-1, 36)
    scale = payload[:, :2].copy().view(np.float16).reshape(-1).astype(np.float64)
    total = payload[:, 2:4].copy().view(np.float16).reshape(-1)
    q = payload[:, 4:].view(np.int8).astype(np.int64)
    amax = np.abs(values).max(axis=1).astype(np.float64)
    exact = amax / 127.0
    near = exact.astype(np.float16).astype(np.float64)
    scale_ok = (scale == near) | (np.abs(scale - near) <= np.spacing(np.float16(near)).astype(np.float64) * 1.01) & \
        (np.abs(exact - (scale + near) / 2) <= 4 * np.spacing(exact.astype(np.float32)).astype(np.float64))
    with np.errstate(invalid="ignore", divide="ignore"):
        target = np.where(amax[:, None] > 0, values.astype(np.float64) * 127.0 / amax[:, None], 0.0)
    nearest = np.copysign(np.floor(np.abs(target) + 0.5), target)
    frac = np.abs(target) - np.floor(np.abs(target))
    tie = np.abs(frac - 0.5) <= 4 * np.abs(np.spacing(target.astype(np.float32))).astype(np.float64)
    code_ok = (q == nearest) | (tie & (np.abs(q - nearest) == 1))
    lanes = values.copy()
    idx = np.arange(32)
    for off in (16, 8, 4, 2, 1):
        lanes = (lanes + lanes[:, idx ^ off]).astype(np.float32)
    sum_ok = total.view(np.uint16) == lanes[:, 0].astype(np.float16).view(np.uint16)
    zero = amax == 0
    scale_ok &= ~zero | (scale == 0)
    code_ok[zero] = q[zero] == 0
    return bool(scale_ok.all()), bool(code_ok.all()), bool(sum_ok.all())


def test_q8_1_known_answer(oracle):
    case = GOLDEN["q8_1"][0]
    x = np.zeros((1, 32), np.float32)
    x[0, :3] = case["block"]
    blk = oracle.quantize(oracle.Q8_1, x)[0]
    assert blk.size == case["block_bytes"]
    assert blk[0:2].view(np.float16)[0] == np.float16(case["scale_f16"])
    assert blk[2:4].view(np.float16)[0] == np.float16(case["sum_f16"])   # original values, not codes
    assert blk[4:7].view(np.int8).tolist() == case["codes"]


def test_q8_1_follows_the_staging_rules(oracle):
    rng = np.random.default_rng(17)
    x = rng.standard_normal((64, 256)).astype(np.float32) * (10.0 ** rng.uniform(-6, 3, (64, 1))).astype(np.float32)
    x[3] = 0
    x[5, :32] = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5] + [0.0] * 25
    # a sum whose F32 value depends on the reduction order: 2048 + 2^-13 is
    # a tie that rounds back to 2048, so only the butterfly that pairs lane 0
    # with lane 16 first keeps the 2^-13
    x[6, :32] = 0
    x[6, 0], x[6, 16], x[6, 1] = 2048.0, -2048.0, 2.0 ** -13
    packed = oracle.quantize(oracle.Q8_1, x)
    assert _q8_1_rules(x, packed) == (True, True, True)
    assert packed[6].reshape(-1, 36)[0, 2:4].view(np.float16)[0] == np.float16(2.0 ** -13)
    # ggml-cuda's quantize_q8_1 rounds with roundf: ties away from zero
    assert packed[5, 4:11].view(np.int8).tolist() == [127, 1, -1, 2, -2, 3, -3]
    bad = oracle.quantize(oracle.Q8_1, x).copy()
    bad[0, 4] ^= 1                                      # a corrupted code fails the rules
    assert not _q8_1_rules(x, bad)[1]


def _mmq_decode(payload, rows, width):
    kp = (width + 511) // 512 * 512
    p = np.asarray(payload, np.uint8).reshape(kp // 128, rows, 144)
    scales = p[:, :, :16].copy().view(np.float32).reshape(-1, rows, 4)
    codes = p[:, :, 16:].view(np.int8).reshape(-1, rows, 4, 32).astype(np.float32)
    values = (scales[:, :, :, None] * codes).transpose(1, 0, 2, 3).reshape(rows, kp)
    return values[:, :width]


def test_q8_1_mmq_known_answers(oracle):
    g = GOLDEN["q8_1_mmq_d4"]
    x = np.zeros((1, 32), np.float32)
    x[0, :7] = g["ties_and_signs"]["block"]
    assert _mmq_decode(oracle.quantize_q8_1_mmq(x), 1, 32)[0, :7].tolist() == g["ties_and_signs"]["decoded"]
    src = np.zeros((3, 256), np.float32)
    src[0] = np.tile(np.arange(-16, 16, dtype=np.float32), 8)
    src[0, ::32] = 127.0
    src[2] = -src[0] * 0.5
    payload = oracle.quantize_q8_1_mmq(src)
    assert payload.size == 4 * 3 * 144                 # 256 values pad to one 512-value row
    assert np.array_equal(_mmq_decode(payload, 3, 256), src)
    tail = ((np.arange(3 * 128, dtype=np.float32).reshape(3, 128) % 53 - 26) * np.float32(0.013))[:, ::2]
    payload = oracle.quantize_q8_1_mmq(tail)
    assert payload.size == 4 * 3 * 144
    dec = _mmq_decode(payload, 3, 64)
    assert np.abs(dec - tail).max() <= np.abs(tail).max() / 127 / 2 * 1.0001


def test_q8_1_mmq_follows_the_staging_rules(oracle):
    # tools/validation/verify_q8_mmq_rhs_staging.py:24-65: F32 scales within
    # 4 ulps of amax/127, codes nearest (half away) or adjacent at ties
    rng = np.random.default_rng(23)
    x = rng.standard_normal((9, 640)).astype(np.float32) * (10.0 ** rng.uniform(-5, 5, (9, 1))).astype(np.float32)
    x[2, 128:256] = 0
    payload = oracle.quantize_q8_1_mmq(x)
    kp = 1024
    p = payload.reshape(kp // 128, 9, 144)
    scales = p[:, :, :16].copy().view(np.float32).reshape(kp // 128, 9, 4).transpose(1, 0, 2).reshape(9, -1)
    codes = p[:, :, 16:].view(np.int8).reshape(kp // 128, 9, 4, 32).transpose(1, 0, 2, 3).reshape(9, -1, 32)
    src = np.zeros((9, kp), np.float32)
    src[:, :640] = x
    blocks = src.reshape(9, -1, 32).astype(np.float64)
    amax = np.abs(blocks).max(axis=2)
    exact = amax / 127.0
    assert (np.abs(scales - exact) <= 4 * np.spacing(exact.astype(np.float32)).astype(np.float64)).all()
    with np.errstate(invalid="ignore", divide="ignore"):
        target = np.where(amax[:, :, None] > 0, blocks * 127.0 / amax[:, :, None], 0.0)
    nearest = np.copysign(np.floor(np.abs(target) + 0.5), target)
    frac = np.abs(target) - np.floor(np.abs(target))
    tie = np.abs(frac - 0.5) <= 4 * np.abs(np.spacing(target.astype(np.float32))).astype(np.float64)
    q = codes.astype(np.int64)
    assert ((q == nearest) | (tie & (np.abs(q - nearest) == 1))).all()
    assert (q[amax == 0] == 0).all() and (scales[amax == 0] == 0).all()


def test_q8_rhs_range_rule(oracle):
    g = GOLDEN["q8_1_mmq_d4"]
    named = {"nan": np.nan, "inf": np.inf, "-inf": -np.inf, "float32_tiny": np.finfo(np.float32).tiny}
    for (v,) in g["fails_closed"]:
        with np.errstate(over="ignore"):
            x = np.full((1, 32), named.get(v, v), dtype=np.float32) if not isinstance(v, str) or v in named else None
        assert not oracle.q8_rhs_supported(x), v
    for v in g["passes"]:
        assert oracle.q8_rhs_supported(np.full((1, 32), v, np.float32)), v
    x = np.ones((2, 64), np.float32)
    x[1, 40] = 1e-31                                   # not a block maximum: passes
    assert oracle.q8_rhs_supported(x)
    x[1, 32:64] = 1e-31                                # block maximum below 1e-30: fails
    assert not oracle.q8_rhs_supported(x)
