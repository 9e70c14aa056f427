"""Write the golden vectors under tests/golden/ from the reference itself.

Run in the build container only, where the mlsquare/coset tree is mounted:

    python tests/golden/make_goldens.py --reference /root/reference

It imports the reference (pure Python/PyTorch, CPU) and records inputs and
outputs of the functions whose bits no closed form fixes: the core
projection with its g_x rule and tie handling (coset/core/e8/lattice.py:
67-169), the legacy Q (coset/legacy/lattices/e8.py:41-103), e8_encode /
e8_decode / e8_quantize (coset/core/e8/codecs.py:17-286), the QAT layer
forward/backward and beta pipeline (coset/core/layers.py:381-478,
coset/core/e8/layers.py:15-66), the legacy one-sided vLUT
(coset/legacy/quant/vlut.py:72-117) and the legacy hierarchical encode /
decode with the overload loop (coset/legacy/quant/functional.py:15-181).
Only data is written (npz, no pickles); nothing here is needed at run time.
--only picks sections (projection, residual, codec, layer, vlut, legacy,
extra); "extra" writes layer_stats.npz (a layer run across its 256th step,
coset/core/layers.py:366-379, 408-413), d4.npz (coset/core/d4/lattice.py:
62-146 and the D4 layer of coset/core/d4/layers.py:14-68) and lsq.npz
(LSQActivation, coset/core/layers.py:117-137).
"""
from __future__ import annotations

import argparse
import os
import sys
import warnings

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def adversarial_blocks(rng: np.random.Generator) -> np.ndarray:
    """Blocks that hit exact ties, grids, zeros and near-equidistant cosets."""
    out = []
    # exact half-integer ties, small and large magnitude (eps nudge vanishes
    # for |x| >= 2)
    out.append(rng.integers(-8, 9, size=(512, 8)) / 2.0)
    out.append(rng.integers(-32, 33, size=(512, 8)) / 4.0)
    out.append(rng.integers(-64, 65, size=(512, 8)) / 8.0)
    out.append(rng.integers(-16, 17, size=(256, 8)) / 2.0 + 0.0)
    # a single tied coordinate in otherwise generic blocks
    g = rng.standard_normal((512, 8))
    j = rng.integers(0, 8, size=512)
    g[np.arange(512), j] = rng.integers(-6, 7, size=512) + 0.5
    out.append(g)
    # several coordinates sharing the same fractional distance (argmax ties)
    base = rng.integers(-3, 4, size=(512, 8)).astype(np.float64)
    frac = rng.choice([0.25, 0.3, 0.45, 0.5], size=(512, 1))
    sgn = rng.choice([-1.0, 1.0], size=(512, 8))
    mask = rng.random((512, 8)) < 0.5
    out.append(base + np.where(mask, sgn * frac, 0.1 * rng.standard_normal((512, 8))))
    # zeros, signed zeros, exact E8 points
    z = np.zeros((8, 8))
    z[1::2] = -0.0
    out.append(z)
    out.append(np.array([[0.25] * 8, [-0.25] * 8, [0.5] * 8, [-0.5] * 8,
                         [0.75] * 8, [1.0] + [0.0] * 7, [0.5] * 4 + [-0.5] * 4,
                         [1.5] * 8, [-1.5] * 8, [2.5] * 8, [-2.5] * 8]))
    # values just off the half-integers by one or a few fp32 ulps
    h = (rng.integers(-6, 7, size=(512, 8)) + 0.5).astype(np.float32)
    steps = rng.integers(-3, 4, size=(512, 8)).astype(np.int32)
    hb = h.view(np.int32) + steps
    out.append(hb.view(np.float32).astype(np.float64))
    # near-equidistant between the D8 and D8+1/2 candidates: points on the
    # bisector of two candidate sets, then jittered at fp32 resolution
    x = rng.standard_normal((1024, 8))
    y0 = np.round(x)
    odd = (y0.sum(axis=1) % 2) != 0
    k = np.argmax(np.abs(x - y0), axis=1)
    y0[odd, k[odd]] += np.where(x[odd, k[odd]] > y0[odd, k[odd]], 1.0, -1.0)
    y1 = np.floor(x) + 0.5
    odd1 = (np.floor(x).sum(axis=1) % 2) != 0
    k1 = np.argmax(np.abs(x - y1), axis=1)
    y1[odd1, k1[odd1]] += np.where(x[odd1, k1[odd1]] > y1[odd1, k1[odd1]], 1.0, -1.0)
    d = y1 - y0
    dd = (d * d).sum(axis=1, keepdims=True)
    t = (((y1 * y1).sum(axis=1, keepdims=True) - (y0 * y0).sum(axis=1, keepdims=True)) / 2
         - (x * d).sum(axis=1, keepdims=True)) / np.where(dd == 0, 1, dd)
    xb = (x + t * d).astype(np.float32)
    jit = rng.integers(-2, 3, size=xb.shape).astype(np.int32)
    out.append((xb.view(np.int32) + jit).view(np.float32).astype(np.float64))
    out.append(xb.astype(np.float64))
    return np.concatenate(out, axis=0).astype(np.float32)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--out", default=HERE)
    ap.add_argument("--only", default="", help="comma list of sections (default: all)")
    args = ap.parse_args()
    only = set(filter(None, args.only.split(",")))
    if only == {"legacy"}:
        return legacy_functional(args)
    if only == {"extra"}:
        return extra_goldens(args)

    sys.path.insert(0, args.reference)
    warnings.simplefilter("ignore")
    import torch
    from coset.core.base import LatticeConfig
    from coset.core.e8.lattice import E8Lattice
    from coset.core.e8.codecs import e8_encode, e8_decode, e8_quantize
    from coset.core.e8.layers import create_e8_hnlq_linear
    from coset.legacy.lattices.e8 import E8Lattice as LegacyE8Lattice
    from coset.legacy.quant.params import QuantizationConfig
    from coset.legacy.quant.vlut import vLUTManager

    torch.set_num_threads(8)
    meta = f"torch {torch.__version__}; generated by tests/golden/make_goldens.py"
    rng = np.random.default_rng(20261201)
    lat = E8Lattice()

    # ---------------- projection / custom_round / g_x ------------------
    adv = adversarial_blocks(rng)
    rnd = np.concatenate([
        rng.standard_normal((4096, 8)).astype(np.float32),
        (0.25 * rng.standard_normal((1024, 8))).astype(np.float32),
        (4.0 * rng.standard_normal((1024, 8))).astype(np.float32),
        (32.0 * rng.standard_normal((512, 8))).astype(np.float32),
    ])
    xs = np.concatenate([adv, rnd])
    xt = torch.from_numpy(xs)
    proj = _np(lat.projection(xt))
    gx = _np(lat.g_x(xt))
    cr = _np(lat.custom_round(xt))
    leg = LegacyE8Lattice()
    sub = xs[:: 7]
    legq = np.stack([_np(leg.Q(torch.from_numpy(v.copy()))) for v in sub])
    np.savez_compressed(os.path.join(args.out, "projection.npz"), x=xs, projection=proj,
                        g_x=gx, custom_round=cr, legacy_x=sub, legacy_q=legq, meta=meta)
    print("projection", xs.shape)

    # ---------------- exhaustive single-level residual tables -----------
    res = {}
    for q in (2, 3, 4):
        b = torch.cartesian_prod(*[torch.arange(q) for _ in range(8)]).float()
        cfg = LatticeConfig(lattice_type="E8", q=q, M=1, beta=1.0)
        r = _np(e8_decode(b.view(-1, 1, 8), cfg))
        two_r = np.rint(2 * r)
        assert np.array_equal(two_r / 2, r)
        res[f"q{q}"] = two_r.astype(np.int8)
    b16 = rng.integers(0, 16, size=(8192, 8))
    cfg = LatticeConfig(lattice_type="E8", q=16, M=1, beta=1.0)
    r16 = _np(e8_decode(torch.from_numpy(b16).float().view(-1, 1, 8), cfg))
    np.savez_compressed(os.path.join(args.out, "residual_tables.npz"),
                        two_r_q2=res["q2"], two_r_q3=res["q3"], two_r_q4=res["q4"],
                        b_q16=b16.astype(np.int8), r_q16=r16.astype(np.float32), meta=meta)
    print("residual tables")

    # ---------------- e8_encode / e8_decode ------------------------------
    enc_cases = {}
    cases = [("q4M2_b1", 4, 2, 1.0), ("q4M2_b025", 4, 2, 0.25), ("q4M2_b03", 4, 2, 0.3),
             ("q4M2_b002", 4, 2, 0.02), ("q16M3_b1", 16, 3, 1.0), ("q3M2_b1", 3, 2, 1.0),
             ("q8M2_b05", 8, 2, 0.5), ("q2M4_b1", 2, 4, 1.0)]
    for name, q, M, beta in cases:
        x = rng.standard_normal((2048, 8)).astype(np.float32)
        if beta == 0.02:
            x = (0.02 * x).astype(np.float32)
        x = np.concatenate([x, adv[:: 5] * np.float32(max(beta, 0.25))]).astype(np.float32)
        t3 = np.clip(rng.standard_t(3, size=(512, 8)), -2, 2).astype(np.float32)
        x = np.concatenate([x, t3]).astype(np.float32)
        cfg = LatticeConfig(lattice_type="E8", q=q, M=M, beta=beta)
        codes, T = e8_encode(torch.from_numpy(x), cfg)
        assert T == 0
        dec = e8_decode(codes, cfg)
        enc_cases[f"{name}_x"] = x
        enc_cases[f"{name}_codes"] = np.rint(_np(codes)).astype(np.int8)
        enc_cases[f"{name}_dec"] = _np(dec)
    xq = rng.standard_normal((1024, 8)).astype(np.float32)
    enc_cases["quantize_x"] = xq
    enc_cases["quantize_q4"] = _np(e8_quantize(torch.from_numpy(xq), q=4))
    enc_cases["quantize_q16"] = _np(e8_quantize(torch.from_numpy(xq), q=16))
    enc_cases["single_x"] = xq[0]
    enc_cases["single_codes"] = np.rint(_np(e8_encode(torch.from_numpy(xq[0]),
                                        LatticeConfig(lattice_type="E8", q=4, M=2))[0])).astype(np.int8)
    np.savez_compressed(os.path.join(args.out, "codec.npz"), meta=meta, **enc_cases)
    print("codec")

    # ---------------- QAT layer forward/backward -------------------------
    lay = {}
    layer_cases = [
        # name, in, out, kwargs, W std, theta
        ("c1", 768, 10, dict(q=4, M=2, theta_init_value=0.0, weight_clip_value=2.0), 0.02, None),
        ("c1nd", 768, 10, dict(q=4, M=2, Delta0=1.5, weight_clip_value=2.0), 1.0, None),
        ("rnd", 64, 16, dict(q=4, M=2, Delta0=1.5, weight_clip_value=2.0), 1.0, "uniform"),
        ("clip", 64, 16, dict(q=4, M=2, Delta0=6.0, weight_clip_value=0.5), 1.0, "uniform"),
        ("q16", 64, 8, dict(q=16, M=3, Delta0=1.5, weight_clip_value=2.0), 1.0, "uniform"),
    ]
    for name, fin, fout, kw, wstd, theta in layer_cases:
        torch.manual_seed(hash(name) % 1000)
        layer = create_e8_hnlq_linear(fin, fout, **kw)
        W = (wstd * rng.standard_normal((fout, fin))).astype(np.float32)
        layer.weight.data = torch.from_numpy(W.copy())
        if theta == "uniform":
            th = rng.uniform(-3, 3, size=fout).astype(np.float32)
            layer.theta_beta.data = torch.from_numpy(th)
        bias = (0.1 * rng.standard_normal(fout)).astype(np.float32)
        layer.bias.data = torch.from_numpy(bias)
        x = rng.standard_normal((32, fin)).astype(np.float32)
        g = rng.standard_normal((32, fout)).astype(np.float32)
        bmin, bmax = layer._bounds()
        beta = bmin + torch.sigmoid(layer.theta_beta) * (bmax - bmin)
        xt = torch.from_numpy(x).requires_grad_(True)
        y = layer(xt)
        (y * torch.from_numpy(g)).sum().backward()
        with torch.no_grad():
            layer.step_count.zero_()
            Wq = layer._quantize_weights()
        for k, v in dict(W=W, bias=bias, x=x, g=g, y=_np(y), Wq=_np(Wq),
                         beta=_np(beta), beta_min=_np(bmin), beta_max=_np(bmax),
                         theta=_np(layer.theta_beta), dW=_np(layer.weight.grad),
                         dtheta=_np(layer.theta_beta.grad), dbias=_np(layer.bias.grad),
                         dx=_np(xt.grad), Delta0=np.float64(layer.Delta0),
                         q=np.int64(layer.q), M=np.int64(layer.M),
                         clip=np.float64(layer.weight_clip_value)).items():
            lay[f"{name}_{k}"] = v
    np.savez_compressed(os.path.join(args.out, "layer.npz"), meta=meta, **lay)
    print("layer")

    # ---------------- legacy one-sided vLUT -------------------------------
    vl = {}
    for q in (3, 4):
        cfg = QuantizationConfig(lattice_type="E8", q=q, M=2)
        mgr = vLUTManager(leg, cfg)
        for i in range(2):
            a = (2.0 * rng.standard_normal(8)).astype(np.float32)
            v = mgr.build_one_sided_vlut(torch.from_numpy(a))
            vl[f"q{q}_a{i}"] = a
            vl[f"q{q}_vlut{i}"] = _np(v)
    np.savez_compressed(os.path.join(args.out, "vlut_legacy.npz"), meta=meta, **vl)
    print("vlut")


def _layer_record(out, name, layer, W, bias, x, g, extra=None):
    """Inputs and outputs of one reference layer step (forward, backward) and
    the beta it used."""
    import torch
    xt = torch.from_numpy(x).requires_grad_(True)
    y = layer(xt)
    (y * torch.from_numpy(g)).sum().backward()
    with torch.no_grad():   # the bounds the step used (after its statistics update, if any)
        bmin, bmax = layer._bounds()
        beta = bmin + torch.sigmoid(layer.theta_beta) * (bmax - bmin)
    rec = dict(W=W, bias=bias, x=x, g=g, y=_np(y), beta=_np(beta), beta_min=_np(bmin), beta_max=_np(bmax),
               theta=_np(layer.theta_beta), dW=_np(layer.weight.grad), dtheta=_np(layer.theta_beta.grad),
               dbias=_np(layer.bias.grad), dx=_np(xt.grad), Delta0=np.float64(layer.Delta0),
               q=np.int64(layer.q), M=np.int64(layer.M), clip=np.float64(layer.weight_clip_value))
    rec.update(extra or {})
    for k, v in rec.items():
        out[f"{name}_{k}"] = v


def extra_goldens(args):
    """Reference outputs for the statistics update, D4 and LSQ."""
    sys.path.insert(0, args.reference)
    warnings.simplefilter("ignore")
    import torch
    from coset.core.e8.layers import create_e8_hnlq_linear
    from coset.core.d4.lattice import D4Lattice
    from coset.core.d4.layers import create_d4_hnlq_linear
    from coset.core.layers import LSQActivation

    torch.set_num_threads(8)
    meta = f"torch {torch.__version__}; generated by tests/golden/make_goldens.py --only extra"
    rng = np.random.default_rng(20261203)

    # ---- layer statistics: 255 forwards, then step 256 (the EMA update runs
    # before the bounds, layers.py:408-413) with forward and backward
    st = {}
    stat_cases = [
        ("row", 64, 16, dict(q=4, M=2, Delta0=1.5, tiling="row")),
        ("c1", 768, 10, dict(q=4, M=2)),
    ]
    for name, fin, fout, kw in stat_cases:
        torch.manual_seed(1)
        layer = create_e8_hnlq_linear(fin, fout, **kw)
        scale = 0.02 if name == "c1" else 1.0
        W = (scale * rng.standard_normal((fout, fin)) * rng.uniform(0.3, 3.0, size=(fout, 1))
             + 0.05 * scale * rng.standard_normal((fout, 1))).astype(np.float32)
        layer.weight.data = torch.from_numpy(W.copy())
        th = rng.uniform(-2, 2, size=layer.theta_beta.numel()).astype(np.float32)
        layer.theta_beta.data = torch.from_numpy(th)
        bias = (0.1 * rng.standard_normal(fout)).astype(np.float32)
        layer.bias.data = torch.from_numpy(bias)
        x = rng.standard_normal((16, fin)).astype(np.float32)
        g = rng.standard_normal((16, fout)).astype(np.float32)
        with torch.no_grad():
            for _ in range(255):
                layer(torch.from_numpy(x))
        assert int(layer.step_count) == 255
        sig0, xm0 = _np(layer.sigma_ema).copy(), _np(layer.xmax_ema).copy()
        _layer_record(st, name, layer, W, bias, x, g)
        assert int(layer.step_count) == 256
        with torch.no_grad():
            Wq = layer._quantize_weights()       # step 257: the statistics stay
        st[f"{name}_sigma_ema_255"] = sig0
        st[f"{name}_xmax_ema_255"] = xm0
        st[f"{name}_sigma_ema"] = _np(layer.sigma_ema)
        st[f"{name}_xmax_ema"] = _np(layer.xmax_ema)
        st[f"{name}_Wq"] = _np(Wq)
        print("stats", name, "sigma moved:", float(np.abs(st[f"{name}_sigma_ema"] - sig0).max()))
    # block tiling: the reference's forward cannot run it (layers.py:459
    # reshapes [out, bpr, 1] to [out, in]), so its _gather_stats is called on
    # the blocks directly, twice (two EMA steps)
    torch.manual_seed(1)
    layer = create_e8_hnlq_linear(32, 8, q=4, M=2, Delta0=1.5, tiling="block")
    W = (rng.standard_normal((8, 32)) * rng.uniform(0.3, 3.0, size=(8, 1))).astype(np.float32)
    st["block_W"] = W
    for i in range(2):
        layer._gather_stats(torch.from_numpy(W).view(8, 4, 8))
        st[f"block_sigma_ema_{i + 1}"] = _np(layer.sigma_ema).copy()
        st[f"block_xmax_ema_{i + 1}"] = _np(layer.xmax_ema).copy()
    np.savez_compressed(os.path.join(args.out, "layer_stats.npz"), meta=meta, **st)

    # ---- D4: projection and g_x (random, ties, half-integers), layer steps
    d4 = {}
    lat = D4Lattice()
    xs = np.concatenate([
        rng.standard_normal((2048, 4)),
        4.0 * rng.standard_normal((512, 4)),
        rng.integers(-8, 9, size=(512, 4)) / 2.0,
        rng.integers(-16, 17, size=(512, 4)) / 4.0,
        np.round(rng.standard_normal((512, 4)) * 4) / 4 + rng.choice([0.0, 1e-7, -1e-7], size=(512, 4)),
    ]).astype(np.float32)
    xt = torch.from_numpy(xs)
    d4["x"] = xs
    d4["projection"] = _np(lat.projection(xt))
    d4["g_x"] = _np(lat.g_x(xt))
    d4_cases = [
        ("d4def", 64, 16, dict(q=4, M=2), 0.02, None),
        ("d4nd", 64, 16, dict(q=4, M=2, Delta0=1.5), 1.0, "uniform"),
        ("d4clip", 32, 8, dict(q=4, M=2, Delta0=6.0, weight_clip_value=0.5), 1.0, "uniform"),
    ]
    for name, fin, fout, kw, wstd, theta in d4_cases:
        torch.manual_seed(2)
        layer = create_d4_hnlq_linear(fin, fout, **kw)
        W = (wstd * rng.standard_normal((fout, fin))).astype(np.float32)
        layer.weight.data = torch.from_numpy(W.copy())
        if theta == "uniform":
            layer.theta_beta.data = torch.from_numpy(
                rng.uniform(-3, 3, size=layer.theta_beta.numel()).astype(np.float32))
        bias = (0.1 * rng.standard_normal(fout)).astype(np.float32)
        layer.bias.data = torch.from_numpy(bias)
        x = rng.standard_normal((16, fin)).astype(np.float32)
        g = rng.standard_normal((16, fout)).astype(np.float32)
        _layer_record(d4, name, layer, W, bias, x, g)
        with torch.no_grad():
            layer.step_count.zero_()
            d4[f"{name}_Wq"] = _np(layer._quantize_weights())
        print("d4", name)
    np.savez_compressed(os.path.join(args.out, "d4.npz"), meta=meta, **d4)

    # ---- LSQ activation quantizer: forward and both gradients
    lsq = {}
    lsq_cases = [("b8_a1", 8, 1.0, 1.0), ("b8_a03", 8, 0.3, 1.0), ("b4_a2", 4, 2.0, 3.0),
                 ("b8_neg", 8, -0.5, 1.0), ("b2_a1", 2, 1.0, 1.5)]
    for name, bits, alpha, xs_scale in lsq_cases:
        q = LSQActivation(bit_width=bits, init_alpha=alpha)
        x = (xs_scale * rng.standard_normal((64, 48))).astype(np.float32)
        x[0, :8] = np.array([0.0, -0.0, alpha, -alpha, 2 * alpha, -2 * alpha, alpha / 3, 1e-9], np.float32)
        g = rng.standard_normal(x.shape).astype(np.float32)
        xt = torch.from_numpy(x).requires_grad_(True)
        y = q(xt)
        (y * torch.from_numpy(g)).sum().backward()
        for k, v in dict(x=x, g=g, y=_np(y), dx=_np(xt.grad), dalpha=_np(q.alpha.grad).reshape(1),
                         alpha=np.array([alpha], np.float32), bits=np.int64(bits)).items():
            lsq[f"{name}_{k}"] = v
    np.savez_compressed(os.path.join(args.out, "lsq.npz"), meta=meta, **lsq)
    print("lsq")


def legacy_functional(args):
    """coset/legacy/quant/functional.py:15-181: per-block encode (with the
    2^alpha overload loop), the final chain's overload flag
    (_encode_internal, 83-116) and decode, one 8-vector per call as the
    reference takes it."""
    sys.path.insert(0, args.reference)
    warnings.simplefilter("ignore")
    import torch
    from coset.legacy.lattices.e8 import E8Lattice as LegacyE8Lattice
    from coset.legacy.quant.params import QuantizationConfig
    from coset.legacy.quant.functional import encode, decode, _encode_internal

    meta = f"torch {torch.__version__}; generated by tests/golden/make_goldens.py --only legacy"
    rng = np.random.default_rng(20261202)
    leg = LegacyE8Lattice()
    cases = [
        ("q4M2_p", dict(q=4, M=2, beta=0.3, alpha=1.0, disable_overload_protection=False)),
        ("q3M2_p", dict(q=3, M=2, beta=0.35, alpha=1.0, disable_overload_protection=False)),
        ("q8M2_a2", dict(q=8, M=2, beta=0.2, alpha=2.0, disable_overload_protection=False)),
        ("q4M3_np", dict(q=4, M=3, beta=0.5, alpha=1.0, disable_overload_protection=True)),
        ("q2M4_p", dict(q=2, M=4, beta=0.4, alpha=1.0, disable_overload_protection=False,
                        max_scaling_iterations=4)),
        ("q4M2_dither", dict(q=4, M=2, beta=0.3, alpha=1.0, disable_overload_protection=False,
                             with_dither=True)),
    ]
    out = {}
    for name, kw in cases:
        cfg = QuantizationConfig(lattice_type="E8", **kw)
        xs = np.concatenate([(s * rng.standard_normal((48, 8))).astype(np.float32)
                             for s in (0.2, 1.0, 3.0, 12.0)])
        dith = (0.01 * rng.standard_normal(8)).astype(np.float32) if cfg.with_dither else None
        codes, Ts, ovs, dec = [], [], [], []
        for v in xs:
            x = torch.from_numpy(v.copy())
            d = torch.from_numpy(dith) if dith is not None else None
            b, T = encode(x, leg, cfg, dither=d)
            xs_t = x / cfg.beta
            if cfg.with_dither and d is not None:
                xs_t = xs_t + d
            for _ in range(T):
                xs_t = xs_t / (2 ** cfg.alpha)
            _, ov = _encode_internal(xs_t, leg, cfg)
            codes.append(_np(b))
            Ts.append(T)
            ovs.append(bool(ov))
            dec.append(_np(decode(b, leg, cfg, T, dither=d)))
        out[f"{name}_x"] = xs
        out[f"{name}_codes"] = np.stack(codes).astype(np.int32)
        out[f"{name}_T"] = np.array(Ts, np.int32)
        out[f"{name}_overload"] = np.array(ovs, np.uint8)
        out[f"{name}_decoded"] = np.stack(dec).astype(np.float32)
        out[f"{name}_cfg"] = np.array([cfg.q, cfg.M, cfg.beta, cfg.alpha, cfg.max_scaling_iterations,
                                       0 if cfg.disable_overload_protection else 1], np.float64)
        if dith is not None:
            out[f"{name}_dither"] = dith
        print(name, "T>0:", int((np.array(Ts) > 0).sum()), "overload:", int(np.sum(ovs)))
    np.savez_compressed(os.path.join(args.out, "legacy_functional.npz"), meta=meta, **out)


if __name__ == "__main__":
    main()
