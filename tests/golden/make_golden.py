"""Writes tests/golden/golden_v1.npz: inputs and expected outputs that pin the
CPU oracle (oracle/oracle.c) independently of it.

Inputs follow the reference's own gate generators: the 64-bit LCG
(x <- 6364136223846793005 x + 1442695040888963407, top bits as the value) with
signed zeros, infinities and NaNs planted every 17th datum
(crates/tt-tests/tests/step61_burn_gather.rs:19-34), and small-integer
matrices whose products are exact in any summation order
(crates/tt-tests/tests/step11_burn.rs:7-10).

Expected outputs come from numpy/scipy in float64, rounded once to float32 --
an implementation independent of the oracle's C code.  Regenerate with
`python tests/golden/make_golden.py` (deterministic).
"""
import os

import numpy as np
from scipy import special

HERE = os.path.dirname(os.path.abspath(__file__))
MASK = (1 << 64) - 1


def lcg_stream(seed, n):
    s = seed | 1
    out = np.empty(n, np.uint64)
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & MASK
        out[i] = s
    return out


def values(seed, n, lo=-4.0, hi=4.0, specials=True):
    """step61's generator: uniform in [lo, hi) from the top 24 bits, with
    -0, +inf, -inf, NaN at i % 17 == 0..3."""
    s = lcg_stream(seed, n)
    v = ((s >> np.uint64(40)).astype(np.float64) / float(1 << 24)) * (hi - lo) + lo
    v = v.astype(np.float32)
    if specials:
        i = np.arange(n)
        v[i % 17 == 0] = -0.0
        v[i % 17 == 1] = np.inf
        v[i % 17 == 2] = -np.inf
        v[i % 17 == 3] = np.nan
    return v


def ints(seed, n, bound):
    s = lcg_stream(seed, n) >> np.uint64(33)
    return ((s % np.uint64(2 * bound + 1)).astype(np.int64) - bound).astype(np.float32)


def f32(x):
    return np.asarray(x, np.float64).astype(np.float32)


def main():
    g = {}
    # ---- element-wise (finite inputs for the transcendental functions)
    x = values(11, 4096, -8.0, 8.0, specials=False)
    xd = x.astype(np.float64)
    g["ew_x"] = x
    g["ew_exp"] = f32(np.exp(xd))
    g["ew_tanh"] = f32(np.tanh(xd))
    g["ew_erf"] = f32(special.erf(xd))
    g["ew_gelu"] = f32(0.5 * xd * special.erfc(-xd / np.sqrt(2.0)))  # 1 + erf without cancellation
    g["ew_sigmoid"] = f32(special.expit(xd))
    g["ew_silu"] = f32(xd * special.expit(xd))  # reference: x * rounded sigmoid
    pos = np.abs(x) + np.float32(1e-3)
    g["ew_pos"] = pos
    g["ew_log"] = f32(np.log(pos.astype(np.float64)))
    g["ew_sqrt"] = f32(np.sqrt(pos.astype(np.float64)))
    g["ew_rsqrt"] = f32(1.0 / np.sqrt(pos.astype(np.float64)))
    gb = values(12, 4096, -2.0, 2.0, specials=False)
    g["ew_g"] = gb
    cdf = 0.5 * (1.0 + special.erf(xd / np.sqrt(2.0)))
    pdf = np.exp(-0.5 * xd * xd) / np.sqrt(2.0 * np.pi)
    g["ew_gelu_bwd"] = f32(gb.astype(np.float64) * (cdf + xd * pdf))
    # GELU's negative tail, where 1 + erf(x / sqrt 2) cancels in float32
    gt = values(19, 512, -12.0, -4.0, specials=False)
    g["ew_gelu_tail_x"] = gt
    g["ew_gelu_tail"] = f32(0.5 * gt.astype(np.float64) * special.erfc(-gt.astype(np.float64) / np.sqrt(2.0)))
    # more transcendental kinds, float64 closed forms rounded once
    g["ew_log1p_x"] = lx = values(15, 4096, -0.9, 8.0, specials=False)
    g["ew_log1p"] = f32(np.log1p(lx.astype(np.float64)))
    g["ew_expm1"] = f32(np.expm1(xd))
    tw = values(16, 4096, -100.0, 100.0, specials=False)
    g["ew_trig_x"] = tw
    g["ew_sin"] = f32(np.sin(tw.astype(np.float64)))
    g["ew_cos"] = f32(np.cos(tw.astype(np.float64)))
    g["ew_pow"] = f32(np.power(pos.astype(np.float64), gb.astype(np.float64)))
    g["ew_pow_s25"] = f32(np.power(pos.astype(np.float64), 2.5))
    g["ew_pow_sm05"] = f32(np.power(pos.astype(np.float64), -0.5))
    g["ew_recip"] = f32(1.0 / xd)
    g["ew_div_s3"] = f32(xd / np.float64(np.float32(3.0)))
    # rsqrt(|x| + 1e-6) as Burn composes it (abs, add_scalar in F32, then the
    # root and reciprocal), with values small enough for the 1e-6 to matter
    ra = np.concatenate([x[:3000], values(17, 1096, -1e-5, 1e-5, specials=False)])
    ra[-4:] = [0.0, -0.0, 1e-30, -1e-6]
    g["ew_rsq_x"] = ra
    t = (np.abs(ra) + np.float32(1e-6)).astype(np.float32)
    g["ew_rsqrt_abs_add"] = f32(1.0 / np.sqrt(t.astype(np.float64)))
    # sigmoid's backward g * s * (1 - s) in Flex's order, two F32 roundings
    # (sfpu/ops.rs:128-130), from a sigmoid output s in (0, 1)
    sg = f32(special.expit(xd))
    g["ew_sig_s"] = sg
    g["ew_sig_bwd"] = ((gb * sg).astype(np.float32) * (np.float32(1.0) - sg)).astype(np.float32)
    g["ew_sig_bwd64"] = f32(gb.astype(np.float64) * sg.astype(np.float64) * (1.0 - sg.astype(np.float64)))
    # exact element-wise ops on special values
    sp = values(13, 1024)
    sq = values(14, 1024)
    g["sp_a"], g["sp_b"] = sp, sq
    with np.errstate(all="ignore"):
        g["sp_add"] = sp + sq
        g["sp_sub"] = sp - sq
        g["sp_mul"] = sp * sq
        g["sp_div"] = sp / sq
        g["sp_relu"] = np.where(sp > 0, sp, np.float32(0.0)).astype(np.float32)
        g["sp_relu_bwd"] = np.where(sp > 0, sq, np.float32(0.0)).astype(np.float32)
        g["sp_gt"] = (sp > sq).astype(np.float32)
        g["sp_eq"] = (sp == sq).astype(np.float32)
        g["sp_neg"] = (sp.view(np.uint32) ^ np.uint32(0x80000000)).view(np.float32)
        g["sp_abs"] = (sp.view(np.uint32) & np.uint32(0x7FFFFFFF)).view(np.float32)
        g["sp_sign"] = np.where(np.isnan(sp), sp, np.where(sp > 0, np.float32(1), np.where(
            sp < 0, np.float32(-1), np.float32(0)))).astype(np.float32)
        # leaky_relu (sfpu/ops.rs:61-62): a >= 0 ? a : slope * a
        g["sp_leaky"] = np.where(sp >= 0, sp, np.float32(0.01) * sp).astype(np.float32)
        # hard_sigmoid (sfpu/ops.rs:63-64): (alpha a + beta).clamp(0, 1), two roundings
        hs = (np.float32(0.2) * sp).astype(np.float32) + np.float32(0.5)
        g["sp_hard_sigmoid"] = np.where(np.isnan(hs), hs, np.minimum(np.maximum(hs, np.float32(0)),
                                                                     np.float32(1))).astype(np.float32)
        # scale_mask_fill (sfpu/ops.rs:246-251): mask ? fill : a * scale
        mk = (lcg_stream(18, 1024) & np.uint64(1)).astype(np.float32)
        g["sp_mask"] = mk
        g["sp_scale_mask_fill"] = np.where(mk != 0, np.float32(-np.inf),
                                           (sp * np.float32(0.125)).astype(np.float32)).astype(np.float32)
        g["sp_div_s0"] = (sp / np.float32(0.0)).astype(np.float32)
    # ---- products: integer-valued (exact) and general (float64 reference)
    ai = ints(21, 37 * 53, 4).reshape(37, 53)
    bi = ints(22, 53 * 29, 4).reshape(53, 29)
    g["mm_ai"], g["mm_bi"] = ai, bi
    g["mm_ci"] = f32(ai.astype(np.float64) @ bi.astype(np.float64))
    a = values(23, 19 * 41, -1.0, 1.0, specials=False).reshape(19, 41)
    b = values(24, 41 * 23, -1.0, 1.0, specials=False).reshape(41, 23)
    g["mm_a"], g["mm_b"] = a, b
    g["mm_c"] = f32(a.astype(np.float64) @ b.astype(np.float64))
    # ---- reductions (float64 sums)
    r = values(31, 33 * 70, -4.0, 4.0, specials=False).reshape(33, 70)
    g["red_x"] = r
    g["red_sum0"] = f32(r.astype(np.float64).sum(axis=0, keepdims=True))
    g["red_sum1"] = f32(r.astype(np.float64).sum(axis=1, keepdims=True))
    g["red_max0"] = r.max(axis=0, keepdims=True)
    g["red_max1"] = r.max(axis=1, keepdims=True)
    g["red_min0"] = r.min(axis=0, keepdims=True)
    g["red_min1"] = r.min(axis=1, keepdims=True)
    g["red_mean_all"] = np.array([f32(r.astype(np.float64).sum()) / np.float32(r.size)], np.float32)
    # ---- softmax / log-softmax, including rows that overflow exp unshifted
    s = values(41, 9 * 130, -30.0, 30.0, specials=False).reshape(9, 130)
    s[0] += np.float32(80.0)
    g["sm_x"] = s
    # Burn's composition: `x - max` and the row sum are F32 tensors
    # (crates/burn-tt/src/ops.rs:5149-5165); each exp and the division or log
    # computed in float64 and rounded once.
    sh = (s - s.max(axis=1, keepdims=True)).astype(np.float32)
    e = np.exp(sh.astype(np.float64))
    ssum = f32(e.sum(axis=1, keepdims=True))
    g["sm_softmax"] = f32(e / ssum.astype(np.float64))
    g["sm_log_softmax"] = (sh - f32(np.log(ssum.astype(np.float64)))).astype(np.float32)
    # ---- norms
    n = values(51, 7 * 96, -3.0, 3.0, specials=False).reshape(7, 96)
    gam = values(52, 96, 0.5, 1.5, specials=False).reshape(1, 96)
    bet = values(53, 96, -0.5, 0.5, specials=False).reshape(1, 96)
    nd = n.astype(np.float64)
    g["nm_x"], g["nm_gamma"], g["nm_beta"] = n, gam, bet
    g["nm_rms"] = f32(nd / np.sqrt((nd * nd).mean(axis=1, keepdims=True) + 1e-5) * gam.astype(np.float64))
    mu = nd.mean(axis=1, keepdims=True)
    var = ((nd - mu) ** 2).mean(axis=1, keepdims=True)
    g["nm_ln"] = f32((nd - mu) / np.sqrt(var + 1e-5) * gam.astype(np.float64) + bet.astype(np.float64))
    # ---- gather, select, argmax (bit-exact by construction)
    t = values(61, 50 * 12)
    t = t.reshape(50, 12)
    idx = (lcg_stream(62, 40) % np.uint64(50)).astype(np.int32)
    g["ix_table"], g["ix_idx"] = t, idx
    g["ix_select"] = t[idx]
    cols = (lcg_stream(63, 50) % np.uint64(12)).astype(np.int32)
    g["ix_cols"] = cols
    g["ix_pick"] = t[np.arange(50), cols].reshape(50, 1)
    am = values(64, 6 * 20, -4.0, 4.0, specials=False).reshape(6, 20)
    am[1, 3] = am[1, 11] = np.float32(9.0)   # tie: first wins
    am[2, 5] = np.nan                          # NaN above every number
    am[2, 7] = np.inf
    am[3] = 0.0
    am[3, 2] = -0.0                            # -0 == +0: first index
    am[4, 19] = np.nan
    am[4, 4] = np.nan                          # first NaN wins
    g["am_x"] = am
    g["am_idx"] = np.array([[int(np.argmax(np.where(np.isnan(row), np.inf, row) if not np.isnan(row).any()
                                        else np.isnan(row)))] for row in am], np.int32)
    np.savez_compressed(os.path.join(HERE, "golden_v1.npz"), **g)
    print("wrote", os.path.join(HERE, "golden_v1.npz"), len(g), "arrays")


if __name__ == "__main__":
    main()
