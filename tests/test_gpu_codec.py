"""Parity of the HIP codec kernels (through the C ABI) with the reference
goldens and the CPU oracle.  Codes bit-exact; decoded values bit-exact too
(the reference decode is exact for q = 2^k and the kernels reproduce its
fp32 operations for every q)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

CODEC_CASES = [("q4M2_b1", 4, 2, 1.0), ("q4M2_b025", 4, 2, 0.25), ("q4M2_b03", 4, 2, 0.3),
               ("q4M2_b002", 4, 2, 0.02), ("q16M3_b1", 16, 3, 1.0), ("q3M2_b1", 3, 2, 1.0),
               ("q8M2_b05", 8, 2, 0.5), ("q2M4_b1", 2, 4, 1.0)]


@pytest.fixture(scope="module")
def ca():
    import coset_amd
    return coset_amd


@pytest.fixture(params=[(1, True), (2, True), (2, False)], ids=["generic", "lut", "lut_general"])
def path(request, ca):
    """Run the test on the generic kernel and on the LDS-table kernel, the
    latter with and without its fixed-format variant (fp32, beta = 2^k)."""
    from coset_amd import _lib
    _lib.require_gpu()
    kernel, plain = request.param
    _lib.set_codec_path(kernel)
    _lib.set_codec_plain(plain)
    yield kernel
    _lib.set_codec_path(0)
    _lib.set_codec_plain(True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def words(t):
    """Packed level words as uint32 numpy (uint16/uint32 tensors copy as is)."""
    return host(t).astype(np.uint32)


def test_projection_golden(ca, golden):
    P = golden("projection")
    lat = ca.E8Lattice()
    np.testing.assert_array_equal(host(lat.projection(dev(P["x"]))), P["projection"])
    np.testing.assert_array_equal(host(lat.g_x(dev(P["x"]))), P["g_x"])
    np.testing.assert_array_equal(host(lat.custom_round(dev(P["x"]))), P["custom_round"])
    leg = ca.LegacyE8Lattice()
    np.testing.assert_array_equal(host(leg.Q(dev(P["legacy_x"]))), P["legacy_q"])


def test_coords_roundtrip(ca):
    lat = ca.E8Lattice()
    rng = np.random.default_rng(5)
    for q in (3, 4, 16):
        z = rng.integers(0, q, size=(1000, 8)).astype(np.float32)
        y = lat.decode_coords(dev(z), q)
        np.testing.assert_array_equal(host(y), O.decode_coords(z.astype(np.int32)))
        np.testing.assert_array_equal(host(lat.encode_coords(y, q)), z)
    # single vector shape is kept
    v = lat.projection(torch.randn(8, device="cuda"))
    assert v.shape == (8,)


@pytest.mark.parametrize("name,q,M,beta", CODEC_CASES)
def test_codec_golden(ca, golden, path, name, q, M, beta):
    C = golden("codec")
    x = C[name + "_x"]
    cfg = ca.LatticeConfig(lattice_type="E8", q=q, M=M, beta=beta)
    codes, T = ca.e8_encode(dev(x), cfg)
    assert T == 0
    np.testing.assert_array_equal(host(codes).astype(np.int32), C[name + "_codes"].astype(np.int32))
    dec = ca.e8_decode(dev(C[name + "_codes"].astype(np.float32)), cfg)
    np.testing.assert_array_equal(host(dec), C[name + "_dec"])
    # packed path: words equal the reference index of each level's digits
    packed = ca.hnlq_encode(dev(x), q, M, beta)
    w = words(packed)
    np.testing.assert_array_equal(w, O.pack_words(C[name + "_codes"], q))
    np.testing.assert_array_equal(host(ca.hnlq_decode(packed, q, M, beta)), C[name + "_dec"])
    pk2, out = ca.hnlq_roundtrip(dev(x), q, M, beta)
    np.testing.assert_array_equal(words(pk2), w)
    np.testing.assert_array_equal(host(out), C[name + "_dec"])


def test_quantize_golden(ca, golden):
    C = golden("codec")
    x = dev(C["quantize_x"])
    for q in (4, 16):
        np.testing.assert_array_equal(host(ca.e8_quantize(x, q)), C[f"quantize_q{q}"])
    codes, _ = ca.e8_encode(dev(C["single_x"]), ca.LatticeConfig(lattice_type="E8", q=4, M=2))
    assert codes.shape == (2, 8)
    np.testing.assert_array_equal(host(codes), C["single_codes"].astype(np.float32))


@pytest.mark.parametrize("q", [2, 3, 4])
def test_exhaustive_single_level_decode(ca, golden, path, q):
    R = golden("residual_tables")
    words = torch.arange(q ** 8, dtype=torch.int64).to(ca.word_dtype(q)).cuda().reshape(-1, 1)
    r = ca.hnlq_decode(words, q, 1, 1.0)
    np.testing.assert_array_equal(np.rint(2 * host(r)).astype(np.int8), R[f"two_r_q{q}"])


def test_q16_decode_sample(ca, golden):
    R = golden("residual_tables")
    cfg = ca.LatticeConfig(lattice_type="E8", q=16, M=1)
    r = ca.e8_decode(dev(R["b_q16"].astype(np.float32).reshape(-1, 1, 8)), cfg)
    np.testing.assert_array_equal(host(r), R["r_q16"])
    # the same codes as packed words go through the short dyadic residual
    w = torch.from_numpy(O.pack_words(R["b_q16"].astype(np.int64).reshape(-1, 1, 8), 16).astype(np.int64))
    rw = ca.hnlq_decode(w.to(ca.word_dtype(16)).cuda().reshape(-1, 1), 16, 1, 1.0)
    np.testing.assert_array_equal(host(rw), R["r_q16"])


@pytest.mark.parametrize("q,n", [(8, 8 ** 8), (16, 1 << 22)])
def test_dyadic_residual_word_decode(ca, q, n):
    """Packed-word decodes at q = 8, 16 take the short dyadic residual
    (residual_dyadic: the CPU checker compares it with the oracle for every
    code at q = 8 and 16); here on the GPU: every q = 8 code and 2^22 random
    q = 16 codes, decoded from packed words, equal the decode of the same
    digits given as float codes (the exact projection path), and a sample
    equals the oracle, over two levels with beta = 0.5."""
    g = torch.Generator(device="cuda").manual_seed(q)
    if q == 8:
        words = torch.arange(n, device="cuda", dtype=torch.int64)
    else:
        words = torch.randint(0, 1 << 32, (n,), device="cuda", generator=g, dtype=torch.int64)
    w2 = torch.stack([words, words.flip(0)], 1)                       # two levels per block
    digits = torch.stack([(w2 >> (4 * (7 - j) if q == 16 else 3 * (7 - j))) & (q - 1) for j in range(8)], -1)
    out_w = ca.hnlq_decode(w2.to(ca.word_dtype(q)), q, 2, 0.5)
    cfg = ca.LatticeConfig(lattice_type="E8", q=q, M=2, beta=0.5)
    out_f = ca.e8_decode(digits.float(), cfg)
    assert torch.equal(out_w.reshape(-1, 8), out_f.reshape(-1, 8))
    sel = torch.randint(0, n, (20000,), device="cuda", generator=g)
    want = O.e8_decode(host(digits[sel]).astype(np.int64), q, 2, beta=0.5)
    np.testing.assert_array_equal(host(out_w.reshape(-1, 8)[sel]), want.reshape(-1, 8))


@pytest.mark.parametrize("n", [0, 1, 2, 255, 257, 1000])
def test_ragged_sizes(ca, path, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, 8)).astype(np.float32)
    for q, M in ((4, 2), (3, 2), (4, 4), (2, 3)):
        pk, out = ca.hnlq_roundtrip(dev(x), q, M, 1.0)
        codes = O.e8_encode(x, q, M)
        np.testing.assert_array_equal(words(pk).reshape(n, M),
                                      O.pack_words(codes, q).reshape(n, M))
        np.testing.assert_array_equal(host(out).reshape(n, 8), O.e8_decode(codes, q, M).reshape(n, 8))


def test_layer_convention_matches_oracle(ca, path):
    """W*beta_row -> quantize -> /beta_row -> clamp (coset/core/layers.py:431-463)."""
    rng = np.random.default_rng(11)
    rows, cols = 48, 256
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    beta = rng.uniform(0.2, 3.0, size=rows).astype(np.float32)
    for q, M, clip in ((4, 2, 2.0), (16, 3, 2.0), (4, 2, 0.3), (4, 1, 2.0), (4, 3, 1.0), (2, 4, 2.0)):
        Wq, qraw, codes = O.layer_quant(W, beta, q, M, clip)
        pk, out = ca.hnlq_roundtrip(dev(W), q, M, beta_row=dev(beta), blocks_per_row=cols // 8,
                                    clip=clip)
        np.testing.assert_array_equal(host(out).reshape(rows, cols), Wq)
        np.testing.assert_array_equal(words(pk),
                                      O.pack_words(codes, q).reshape(-1, M))


def test_bf16_input_heavy_tailed(ca):
    """C3 shape in miniature: Student-t(3) clipped at +-2, bf16 in, q16 M3,
    per-row beta; the kernel upcasts bf16 exactly."""
    rng = np.random.default_rng(12)
    rows, cols = 64, 1024
    x = np.clip(rng.standard_t(3, size=(rows, cols)), -2, 2).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    x_up = xb.float().numpy()
    beta = rng.uniform(2.0, 20.0, size=rows).astype(np.float32)
    Wq, _, codes = O.layer_quant(x_up, beta, 16, 3, 2.0)
    pk, out = ca.hnlq_roundtrip(xb.cuda(), 16, 3, beta_row=dev(beta), blocks_per_row=cols // 8,
                                clip=2.0)
    np.testing.assert_array_equal(host(out).reshape(rows, cols), Wq)
    np.testing.assert_array_equal(words(pk),
                                  O.pack_words(codes, 16).reshape(-1, 3))
    _, outb = ca.hnlq_roundtrip(xb.cuda(), 16, 3, beta_row=dev(beta), blocks_per_row=cols // 8,
                                clip=2.0, out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(host(outb.float()).reshape(rows, cols),
                                  torch.from_numpy(Wq).to(torch.bfloat16).float().numpy())


def test_dither(ca):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((300, 8)).astype(np.float32)
    d = (0.3 * rng.standard_normal(8)).astype(np.float32)
    cfg = ca.LatticeConfig(lattice_type="E8", q=4, M=2, beta=0.5, with_dither=True)
    codes, _ = ca.e8_encode(dev(x), cfg, dither=dev(d))
    xs = (x / np.float32(0.5) + d).astype(np.float32)
    np.testing.assert_array_equal(host(codes).astype(np.int32), O.e8_encode(xs, 4, 2, 1.0))
    # without with_dither the dither is ignored, as in the reference
    cfg2 = ca.LatticeConfig(lattice_type="E8", q=4, M=2, beta=0.5)
    codes2, _ = ca.e8_encode(dev(x), cfg2, dither=dev(d))
    np.testing.assert_array_equal(host(codes2).astype(np.int32), O.e8_encode(x, 4, 2, 0.5))


def test_host_tensors_follow_input_device(ca):
    x = torch.randn(10, 8)
    cfg = ca.LatticeConfig(lattice_type="E8", q=4, M=2)
    codes, _ = ca.e8_encode(x, cfg)
    assert codes.device.type == "cpu"
    np.testing.assert_array_equal(codes.numpy().astype(np.int32), O.e8_encode(x.numpy(), 4, 2))


def test_errors(ca):
    cfg = ca.LatticeConfig(lattice_type="E8", q=4, M=2)
    with pytest.raises(ValueError):
        ca.e8_encode(torch.randn(4, 7, device="cuda"), cfg)
    with pytest.raises(ValueError):
        ca.e8_decode(torch.zeros(4, 2, 8, device="cuda"), cfg, method="fast")
    with pytest.raises(ValueError):
        ca.e8_encode(torch.randn(4, 8, device="cuda"),
                     ca.LatticeConfig(lattice_type="E8", q=17, M=2))


def test_full_size_c2_properties(ca, path):
    """BASELINE C2 at full size (2^24 blocks, q4 M2, beta 1): a random sample
    of blocks against the oracle, and the fused pass equal to encode then
    decode as separate kernels."""
    n = 1 << 24
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn((n, 8), device="cuda", generator=g)
    pk, out = ca.hnlq_roundtrip(x, 4, 2, 1.0)
    idx = torch.randint(0, n, (1 << 15,), device="cuda", generator=g)
    xs = host(x[idx])
    codes = O.e8_encode(xs, 4, 2)
    np.testing.assert_array_equal(words(pk)[host(idx)], O.pack_words(codes, 4))
    np.testing.assert_array_equal(host(out[idx]), O.e8_decode(codes, 4, 2))
    pk2 = ca.hnlq_encode(x, 4, 2, 1.0)
    assert torch.equal(pk2.view(torch.int16), pk.view(torch.int16))
    out2 = ca.hnlq_decode(pk2, 4, 2, 1.0)
    assert torch.equal(out2, out)
    # every decoded block lies in the scaled lattice: 2*out integral
    assert torch.equal(out * 2, torch.round(out * 2))


def _adversarial_blocks(rng, n):
    """Blocks the encoder's fast projection must hand to the exact sequence:
    dyadic grids (ties), values a few ulp from half-integers, points on the
    boundary between the D8 and D8 + 1/2 candidates, large and tiny values,
    mixed with ordinary Gaussian coordinates."""
    fam = []
    fam.append(rng.integers(-8, 9, (n, 8)) / 2.0 ** rng.integers(0, 5, (n, 1)))
    base = 0.5 * rng.integers(-8, 9, (n, 8))
    fam.append(np.nextafter(base.astype(np.float32), np.float32(np.inf) * rng.choice([-1, 1], (n, 8))))
    p = rng.integers(-6, 7, (n, 8)).astype(np.float64)
    p[:, 0] += p.sum(1) % 2
    h = rng.integers(-6, 7, (n, 8)) + 0.5
    h[:, 1] += np.floor(h).sum(1) % 2
    lam = 0.5 + (rng.random((n, 1)) - 0.5) * 1e-5
    fam.append(p + lam * (h - p))
    fam.append(rng.standard_normal((n, 8)) * rng.choice([1e-30, 1e-6, 3e3, 1e6], (n, 1)))
    x = np.concatenate(fam).astype(np.float32)
    mix = rng.random(x.shape) < 0.3
    x[mix] = rng.standard_normal(mix.sum()).astype(np.float32)
    return x


@pytest.mark.parametrize("q,M", [(4, 2), (16, 3), (2, 4)])
def test_fast_projection_same_codes(ca, path, q, M):
    """Encoder codes with the fast projection equal those of the reference
    operation sequence and of the oracle, on Gaussian and adversarial blocks."""
    from coset_amd import _lib
    rng = np.random.default_rng(17 + q)
    x = np.concatenate([rng.standard_normal((20000, 8)).astype(np.float32),
                        _adversarial_blocks(rng, 5000)])
    xd = dev(x)
    try:
        outs = []
        for fast in (True, False):
            _lib.set_fast_projection(fast)
            outs.append(words(ca.hnlq_encode(xd, q, M, 1.0)))
    finally:
        _lib.set_fast_projection(True)
    np.testing.assert_array_equal(outs[0], outs[1])
    ref = O.pack_words(O.e8_encode(x, q, M), q)
    np.testing.assert_array_equal(outs[0], ref)


def _tiny_and_sparse_blocks(rng, n):
    """Blocks whose coordinates sit within 2^-20 of an integer: tiny blocks
    (every level encodes to 0), exact and signed zeros, and zeros among
    ordinary values -- the fast path's condition (3) fails on all of them."""
    scales = np.array([0.12, 1e-2, 1e-4, 1e-6, 9.5e-7, 1e-9, 1e-20, 1e-38, 1e-44], dtype=np.float32)
    tiny = np.clip(rng.standard_normal((n, 8)).astype(np.float32)
                   * scales[rng.integers(0, len(scales), n)][:, None], -0.124, 0.124).astype(np.float32)
    zeros = np.where(rng.random((n, 8)) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    sparse = np.where(rng.random((n, 8)) < 0.6, np.float32(0.0),
                      rng.standard_normal((n, 8)).astype(np.float32) * 3).astype(np.float32)
    near = np.round(rng.standard_normal((n, 8)) * 4).astype(np.float32)
    near += (rng.standard_normal((n, 8)) * 1e-7).astype(np.float32)
    return np.concatenate([tiny, zeros, sparse, near]).astype(np.float32)


@pytest.mark.parametrize("q,M", [(4, 2), (16, 3), (2, 4), (3, 2)])
def test_tiny_and_sparse_blocks(ca, path, q, M):
    """The encoders' fast path with condition (5) (tiny blocks and exact
    zeros decided for the D8 candidate) gives the oracle's codes and decoded
    values, the same as the reference operation sequence; in the codec and
    in the layer convention (W * beta_row, the degenerate C5 setting of
    W ~ N(0, 0.02) with a small beta among the rows)."""
    from coset_amd import _lib
    rng = np.random.default_rng(23 + q + M)
    x = _tiny_and_sparse_blocks(rng, 3000)
    xd = dev(x)
    try:
        outs = []
        for fast in (True, False):
            _lib.set_fast_projection(fast)
            pk, out = ca.hnlq_roundtrip(xd, q, M, 1.0)
            outs.append((words(pk), host(out)))
    finally:
        _lib.set_fast_projection(True)
    codes = O.e8_encode(x, q, M)
    np.testing.assert_array_equal(outs[0][0], O.pack_words(codes, q).reshape(outs[0][0].shape))
    np.testing.assert_array_equal(outs[0][1].reshape(-1, 8), O.e8_decode(codes, q, M).reshape(-1, 8))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])

    rows, cols = 64, 512
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    W[::5, ::3] = 0.0
    beta = np.exp(rng.uniform(np.log(1e-6), np.log(40.0), size=rows)).astype(np.float32)
    Wq, qraw, lcodes = O.layer_quant(W, beta, q, M, 2.0)
    pk, out = ca.hnlq_roundtrip(dev(W), q, M, beta_row=dev(beta), blocks_per_row=cols // 8, clip=2.0)
    np.testing.assert_array_equal(host(out).reshape(rows, cols), Wq)
    np.testing.assert_array_equal(words(pk), O.pack_words(lcodes, q).reshape(-1, M))


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("beta,extra", [(1.0, 0), (0.25, 3), (0.3, 1), (1.0, 2)])
def test_roundtrip_with_float_codes(ca, path, beta, extra, dynamic):
    """One round trip writing packed words, the reference's float code
    tensor and the decoded blocks together (every kernel variant, both
    schedules of the fixed-format kernel); block counts that end inside a
    wave and inside a group of four lanes too (the fixed-format kernel
    writes the codes and the decoded values of a wave's blocks together,
    clamping lanes past the end to the last block)."""
    from coset_amd import _lib
    rng = np.random.default_rng(int(beta * 100) + extra)
    x = np.concatenate([rng.standard_normal((70000 + extra, 8)),
                        _adversarial_blocks(rng, 2000)]).astype(np.float32)
    n = x.shape[0]
    xd = dev(x)
    packed = torch.empty((n, 2), dtype=torch.uint16, device="cuda")
    codes = torch.empty((n, 2, 8), dtype=torch.float32, device="cuda")
    out = torch.empty((n, 8), dtype=torch.float32, device="cuda")
    _lib.set_codec_dynamic(dynamic)
    try:
        _lib.call("coset_e8_hnlq_roundtrip", _lib.ptr(xd), _lib.F32, n, _lib.SCALE_CODEC, beta, None, 0, 0.0,
                  None, 0, 4, 2, 1, _lib.ptr(packed), _lib.ptr(codes), _lib.ptr(out), _lib.F32,
                  _lib.stream_of(xd))
    finally:
        _lib.set_codec_dynamic(True)
    ref = O.e8_encode(x, 4, 2, beta)
    np.testing.assert_array_equal(host(codes).astype(np.int32), ref)
    np.testing.assert_array_equal(words(packed), O.pack_words(ref, 4))
    np.testing.assert_array_equal(host(out), O.e8_decode(ref, 4, 2, beta))


def test_dynamic_schedule_matches_static(ca):
    """The fixed-format table kernel's dynamic tile schedule (a counter pair
    from the per-device ring per launch, reset by the last workgroup) against
    its static grid stride: partial last tiles, fewer tiles than workgroups, calls repeated
    on one stream and interleaved over three streams, all three modes."""
    from coset_amd import _lib
    _lib.require_gpu()
    rng = np.random.default_rng(31)
    streams = [torch.cuda.current_stream(), torch.cuda.Stream(), torch.cuda.Stream()]
    try:
        _lib.set_codec_path(2)
        for n in (1, 1000, 2047, 2049, 300001, (1 << 21) + 5):
            x = dev(rng.standard_normal((n, 8)).astype(np.float32))
            _lib.set_codec_dynamic(False)
            pk_s, out_s = ca.hnlq_roundtrip(x, 4, 2, 1.0)
            enc_s = ca.hnlq_encode(x, 2, 4, 1.0)
            dec_s = ca.hnlq_decode(enc_s, 2, 4, 1.0)
            _lib.set_codec_dynamic(True)
            torch.cuda.synchronize()
            for rep in range(3):
                for s in streams:
                    with torch.cuda.stream(s):
                        pk, out = ca.hnlq_roundtrip(x, 4, 2, 1.0)
                        enc = ca.hnlq_encode(x, 2, 4, 1.0)
                        dec = ca.hnlq_decode(enc, 2, 4, 1.0)
                    s.synchronize()
                    assert torch.equal(pk.view(torch.int16), pk_s.view(torch.int16)), (n, rep)
                    assert torch.equal(out, out_s), (n, rep)
                    assert torch.equal(enc.view(torch.int16), enc_s.view(torch.int16)), (n, rep)
                    assert torch.equal(dec, dec_s), (n, rep)
            k = min(n, 4096)
            xs = host(x[:k])
            codes = O.e8_encode(xs, 4, 2)
            np.testing.assert_array_equal(words(pk)[:k], O.pack_words(codes, 4))
            np.testing.assert_array_equal(host(out[:k]), O.e8_decode(codes, 4, 2))
            # the round trip without packed words, and decodes of 1 and 3 levels
            _, out_np = ca.hnlq_roundtrip(x, 4, 2, 1.0, want_packed=False)
            assert torch.equal(out_np, out_s), n
            for q, M in ((4, 1), (2, 3)):
                pw = ca.hnlq_encode(x, q, M, 1.0)
                _lib.set_codec_dynamic(False)
                dec_static = ca.hnlq_decode(pw, q, M, 1.0)
                _lib.set_codec_dynamic(True)
                assert torch.equal(ca.hnlq_decode(pw, q, M, 1.0), dec_static), (n, q, M)
                c = O.e8_encode(xs, q, M)
                np.testing.assert_array_equal(host(dec_static[:k]), O.e8_decode(c, q, M))
    finally:
        _lib.set_codec_dynamic(True)
        _lib.set_codec_path(0)


def test_fixed_format_kernel_in_a_graph(ca):
    """A round trip captured in a HIP graph (the fixed-format kernel takes the
    static schedule there) replayed three times, with eager calls on the
    capturing stream between the replays: every replay equals the eager
    result, and so does every eager call."""
    from coset_amd import _lib
    _lib.require_gpu()
    n = (1 << 20) + 777
    g = torch.Generator(device="cuda").manual_seed(41)
    x = torch.randn((n, 8), device="cuda", generator=g)
    x2 = torch.randn((n, 8), device="cuda", generator=g)
    pk_ref, out_ref = ca.hnlq_roundtrip(x, 4, 2, 1.0)
    pk_ref2, out_ref2 = ca.hnlq_roundtrip(x2, 4, 2, 1.0)
    pk = torch.empty_like(pk_ref)
    out = torch.empty_like(out_ref)
    pk2 = torch.empty_like(pk_ref)
    out2 = torch.empty_like(out_ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        ca.hnlq_roundtrip(x, 4, 2, 1.0, packed_out=pk, decoded_out=out)   # warm-up on the side stream
        s.synchronize()
        with torch.cuda.graph(graph, stream=s):
            ca.hnlq_roundtrip(x, 4, 2, 1.0, packed_out=pk, decoded_out=out)
    torch.cuda.synchronize()
    for rep in range(3):
        pk.zero_()
        out.zero_()
        graph.replay()
        with torch.cuda.stream(s):
            ca.hnlq_roundtrip(x2, 4, 2, 1.0, packed_out=pk2, decoded_out=out2)
        torch.cuda.synchronize()
        assert torch.equal(pk.view(torch.int16), pk_ref.view(torch.int16)), rep
        assert torch.equal(out, out_ref), rep
        assert torch.equal(pk2.view(torch.int16), pk_ref2.view(torch.int16)), rep
        assert torch.equal(out2, out_ref2), rep


def test_full_size_c3(ca):
    """C3 at full size (4096 x 8192 Student-t(3) clipped at +-2, bf16 in,
    q16 M3, clamp 2) with the config's per-row beta: the a10 bounds with
    Delta0 = 1.5 and the rows' own std and abs-max, sigmoid(theta) uniform in
    (0, 1), as bench.py derives it (beta spans ~3e-4 .. 1e2 on this data).
    48 rows against the oracle bit for bit (decoded values and level words):
    the 8 rows of smallest and of largest beta (where the coarsest levels and
    the clamp bind) and 32 random ones; over every block the clamp bound and
    the lattice property: 2 W_q beta is an integer vector (up to the rounding
    of the division by beta) wherever the clamp did not bind."""
    rows, cols = 4096, 8192
    g = torch.Generator(device="cuda").manual_seed(3)
    z = torch.randn((rows, cols), device="cuda", generator=g)
    chi = (torch.randn((rows, cols, 3), device="cuda", generator=g) ** 2).sum(-1) / 3
    x = torch.clamp(z / chi.sqrt(), -2.0, 2.0).to(torch.bfloat16)
    del z, chi
    xf = x.float()
    sigma = xf.std(dim=1) + 1e-8
    xmax = xf.abs().amax(dim=1) + 1e-8
    del xf
    q, M, Delta0, eta, ginv = 16, 3, 1.5, 0.1, 12.0
    qM = float(q ** M)
    bmin = (Delta0 / qM) / (eta * ginv * sigma)
    bmax = torch.minimum((Delta0 * (qM - 1)) / (2 * ginv * xmax), (Delta0 * (qM - 1)) / (2 * eta * ginv * sigma))
    bmin = torch.minimum(bmin, bmax * 0.9)
    beta = (bmin + torch.rand(rows, device="cuda", generator=g) * (bmax - bmin)).contiguous()
    print(f"C3 beta range {float(beta.min()):.3g} .. {float(beta.max()):.3g}", flush=True)
    n = rows * cols // 8
    pk, out = ca.hnlq_roundtrip(x.reshape(n, 8), 16, 3, beta_row=beta, blocks_per_row=cols // 8, clip=2.0)
    W = out.reshape(rows, cols)
    assert float(W.abs().max()) <= 2.0
    scaled = (W * beta[:, None]).double() * 2.0
    inside = W.abs() < 2.0
    err = (scaled - scaled.round()).abs()
    # one fp32 division's rounding, relative to |2 W beta| (< 2 * 2 * 128)
    assert float(err[inside].max()) < 4e-3
    order = torch.argsort(beta).cpu()
    rnd = torch.randperm(rows, generator=torch.Generator().manual_seed(5))[:32]
    sel = torch.cat([order[:8], order[-8:], rnd])
    xs = x[sel.cuda()].float().cpu().numpy()
    Wq, _, codes = O.layer_quant(xs, host(beta[sel.cuda()]), 16, 3, 2.0)
    np.testing.assert_array_equal(host(W[sel.cuda()]), Wq)
    got = words(pk).reshape(rows, cols // 8, 3)[sel.numpy()]
    np.testing.assert_array_equal(got.reshape(-1, 3), O.pack_words(codes, 16).reshape(-1, 3))


@pytest.mark.parametrize("q", [4, 8, 16])
def test_layer_roundtrip_kernel_matches_generic(ca, q):
    """The layer round-trip kernel (SCALE_LAYER with stored per-row betas,
    q = 4, 8, 16, M <= 4: one reciprocal per block and div_by_recip for
    dec / beta, med3 clamp) bit for bit against the generic kernel
    (set_codec_plain(False)): every M, fp32 and bf16 inputs and outputs,
    rows of 1, 7, 96 and 512 blocks, block counts that end inside a
    workgroup, betas log-uniform over 1e-3 .. 1e3 with the division's edge
    cases (2^-64 and 2^64 and the floats just outside, 0, negative,
    subnormal, huge, inf, NaN), clips of 2, inf and 1e-3; the fp32 outputs
    of finite rows also against the oracle on a sample."""
    from coset_amd import _lib
    rng = np.random.default_rng(40 + q)
    specials = np.array([2.0 ** -64, 2.0 ** 64, np.nextafter(np.float32(2.0 ** -64), np.float32(0)),
                         np.nextafter(np.float32(2.0 ** 64), np.float32(np.inf)), 0.0, -1.5, 1e-40, 3e38,
                         np.inf, np.nan, -np.inf, 1e-20, 1e20, -2.0 ** -64], dtype=np.float32)
    checked = 0
    try:
        for bpr, rows in ((1, 3621), (7, 517), (96, 37), (512, 7)):
            n = bpr * rows
            beta = np.exp(rng.uniform(np.log(1e-3), np.log(1e3), rows)).astype(np.float32)
            k = min(rows // 2, len(specials))
            beta[rng.choice(rows, k, replace=False)] = specials[:k] if rows > 40 else specials[rng.choice(len(specials), k, replace=False)]
            x = (rng.standard_normal((n, 8)) * rng.choice([0.05, 1.0, 30.0], (n, 1))).astype(np.float32)
            x[rng.choice(n, 3, replace=False)] = 0.0
            xd = dev(x)
            bd = dev(beta)
            for M in (1, 2, 3, 4):
                for xdt in (torch.float32, torch.bfloat16):
                    for clip in (2.0, float("inf"), 1e-3):
                        odt = torch.bfloat16 if (M + bpr) % 2 else torch.float32
                        res = []
                        for plain in (True, False):
                            _lib.set_codec_plain(plain)
                            pk, out = ca.hnlq_roundtrip(xd.to(xdt), q, M, beta_row=bd, blocks_per_row=bpr,
                                                        clip=clip, out_dtype=odt)
                            res.append((words(pk), host(out.view(torch.int32 if odt == torch.float32 else torch.int16))))
                        case = f"q={q} M={M} bpr={bpr} x={xdt} out={odt} clip={clip}"
                        np.testing.assert_array_equal(res[0][0], res[1][0], err_msg=case)
                        np.testing.assert_array_equal(res[0][1], res[1][1], err_msg=case)
                        checked += 1
                        if odt == torch.float32 and xdt == torch.float32 and clip == 2.0:
                            # rows whose scaled blocks stay below 2^20 (the reference's fp32
                            # encode_coords is exact there; far beyond it the digits leave
                            # int32 here and the oracle's doubles, and torch's own matmul
                            # rounds): the 2^-64 rows among them
                            big = np.abs(x.reshape(rows, -1).astype(np.float64)).max(1) * np.abs(beta)
                            ok = np.isfinite(beta) & (beta != 0) & (big < 2.0 ** 20)
                            sel = np.concatenate([np.flatnonzero(ok & (np.abs(beta) < 1e-10))[:2],
                                                  np.flatnonzero(ok & (np.abs(beta) >= 1e-10))[:4]])
                            xs = x.reshape(rows, bpr * 8)[sel]
                            Wq, _, codes = O.layer_quant(xs, beta[sel], q, M, 2.0)
                            got = res[0][1].view(np.float32).reshape(rows, bpr * 8)[sel]
                            np.testing.assert_array_equal(got, Wq, err_msg=case)
                            gw = res[0][0].reshape(rows, bpr, M)[sel].reshape(-1, M)
                            np.testing.assert_array_equal(gw, O.pack_words(codes, q).reshape(-1, M), err_msg=case)
    finally:
        _lib.set_codec_plain(True)
    assert checked == 4 * 4 * 2 * 3


def test_input_lengths_are_checked():
    """Lengths the kernels index by are validated on the host: a dither of
    neither 8 nor 8 n values, a per-row beta that does not tile the blocks,
    a vLUT scale or a packed layer's beta/bias of the wrong length."""
    import coset_amd as ca
    x = torch.randn(40, 8, device="cuda")
    with pytest.raises(ValueError):
        ca.hnlq_encode(x, 4, 2, 1.0, dither=torch.zeros(3, 8, device="cuda"))
    ca.hnlq_encode(x, 4, 2, 1.0, dither=torch.zeros(40, 8, device="cuda"))
    with pytest.raises(ValueError):
        ca.hnlq_roundtrip(x, 4, 2, beta_row=torch.ones(3, device="cuda"), blocks_per_row=10)
    with pytest.raises(ValueError):
        ca.hnlq_decode(torch.zeros(40, 2, dtype=torch.uint16, device="cuda"), 4, 2,
                       beta_row=torch.ones(7, device="cuda"))
    words = torch.zeros(16, 4, 2, dtype=torch.uint16, device="cuda")
    a = torch.randn(2, 32, device="cuda").half()
    with pytest.raises(ValueError):
        ca.vlut_matmul(words, a, 4, scale=torch.ones(15, device="cuda"))
    tensors = {"words": words.cpu(), "beta": torch.ones(15)}
    meta = {"q": 4, "M": 2, "in_features": 32, "out_features": 16}
    with pytest.raises(ValueError):
        ca.PackedLinear(tensors, meta)
    with pytest.raises(ValueError):
        ca.PackedLinear({"words": words.cpu(), "beta": torch.ones(16), "bias": torch.zeros(5)}, meta)


def test_dynamic_schedule_on_many_streams(ca):
    """More streams than the old per-stream slot table held (64), each
    launching concurrently with the others, and more launches than one lap
    of the counter ring: every result equals the static schedule's."""
    from coset_amd import _lib
    _lib.require_gpu()
    rng = np.random.default_rng(32)
    x = dev(rng.standard_normal(((1 << 20) + 333, 8)).astype(np.float32))
    try:
        _lib.set_codec_path(2)
        _lib.set_codec_dynamic(False)
        _, ref = ca.hnlq_roundtrip(x, 4, 2, 1.0)
        _lib.set_codec_dynamic(True)
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream() for _ in range(80)]
        outs = []
        for s in streams:
            with torch.cuda.stream(s):
                outs.append(ca.hnlq_roundtrip(x, 4, 2, 1.0)[1])
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert torch.equal(o, ref), i
        # 8300 launches on one stream: past one lap of the ring's 8192 counter pairs
        out = torch.empty_like(ref)
        small = x[:4096]
        _lib.set_codec_dynamic(False)
        _, ref_small = ca.hnlq_roundtrip(small, 4, 2, 1.0)
        _lib.set_codec_dynamic(True)
        for _ in range(8300):
            ca.hnlq_roundtrip(small, 4, 2, 1.0, decoded_out=out[:4096], want_packed=False)
        torch.cuda.synchronize()
        assert torch.equal(out[:4096], ref_small)
    finally:
        _lib.set_codec_dynamic(True)
        _lib.set_codec_path(0)


def test_dynamic_schedule_held_back_launch(ca):
    """A launch queued behind other work on its stream while more than one
    lap of the counter ring's launches start and finish on another stream,
    the last of them large enough to run beside it: the held-back launch
    keeps its counter pair until it has finished, so both results equal the
    static schedule's."""
    from coset_amd import _lib
    _lib.require_gpu()
    rng = np.random.default_rng(33)
    x = dev(rng.standard_normal(((1 << 21) + 77, 8)).astype(np.float32))
    small = x[:2048]
    try:
        _lib.set_codec_path(2)
        _lib.set_codec_dynamic(False)
        _, ref = ca.hnlq_roundtrip(x, 4, 2, 1.0)
        _, ref_small = ca.hnlq_roundtrip(small, 4, 2, 1.0)
        _lib.set_codec_dynamic(True)
        torch.cuda.synchronize()
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        busy = torch.empty(1 << 26, device="cuda")
        out_a = torch.empty_like(ref)
        out_b = torch.empty_like(ref)
        out_s = torch.empty_like(ref_small)
        with torch.cuda.stream(sa):
            for i in range(40):            # ~10 ms of fills ahead of the held-back launch
                busy.fill_(float(i))
            ca.hnlq_roundtrip(x, 4, 2, 1.0, decoded_out=out_a, want_packed=False)
        with torch.cuda.stream(sb):
            for _ in range(8200):
                ca.hnlq_roundtrip(small, 4, 2, 1.0, decoded_out=out_s, want_packed=False)
            ca.hnlq_roundtrip(x, 4, 2, 1.0, decoded_out=out_b, want_packed=False)
        torch.cuda.synchronize()
        assert torch.equal(out_a, ref)
        assert torch.equal(out_b, ref)
        assert torch.equal(out_s, ref_small)
    finally:
        _lib.set_codec_dynamic(True)
        _lib.set_codec_path(0)
