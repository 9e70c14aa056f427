"""vLUT kernels against the reference's legacy one-sided tables
(tests/golden/vlut_legacy.npz), the oracle, and decode-then-dot.

Tolerances are elementwise and relative to the magnitude of the summands
that make up each value: a table entry <a, r(b)> within 1e-6 of
sum_j |a_j| |r_j(b)|; a lookup sum or matmul output within RTOL[method] of
sum_k sum_m q^m |<a_k, r(b_m)>|, bounded by |a| @ (sum_m q^m |r(b_m)|)^T
times the row's scale.  On the matrix cores every product a x 2 x_hat is
exact (both exact in the operand type) and only the fp32 sums round; the
oracle's own sum of fp32 8-term table entries over at most ~1,100 terms
errs by at most ~1,100 ulp of the magnitude, so 2^-14 holds with margin at
the tests' sizes (typical errors are ~2^-20).  The LDS-table method rounds
its pair-table entries once more (2^-12).  The north star's bound, 1e-3,
is far looser than either."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


RTOL = {"mfma": 2.0 ** -14, "lds": 2.0 ** -12, "auto": 2.0 ** -12}


def close(a, b, mag, tol):
    """Elementwise |a - b| <= tol * max(mag, |b|)."""
    a, b, mag = (np.asarray(t, np.float64) for t in (a, b, mag))
    bound = tol * np.maximum(mag, np.abs(b))
    bad = np.abs(a - b) > bound
    assert not bad.any(), (int(bad.sum()), float(np.abs(a - b)[bad].max()), float(bound[bad].min()))


_RTABLES = {}


def abs_residuals(q, legacy):
    """|r(b)| for every level word of q (oracle residual table), float64."""
    key = (q, bool(legacy))
    if key not in _RTABLES:
        _RTABLES[key] = np.abs(O.residual_table(q, legacy=legacy).astype(np.float64))
    return _RTABLES[key]


def matmul_mag(words_np, q, M, act, scale=None, scale_mode=0, legacy=False):
    """Bound of the summands' magnitude of every vLUT matmul output:
    |a| @ (sum_m q^m |r(b_m)|)^T, times |s_o| (or / |s_o| for scale_mode 1)."""
    R = abs_residuals(q, legacy)
    rows, kb, _ = words_np.shape
    w = np.zeros((rows, kb, 8))
    for m in range(M):
        w += float(q) ** m * R[np.asarray(words_np[:, :, m], np.int64)]
    mag = np.abs(np.asarray(act, np.float64)) @ w.reshape(rows, kb * 8).T
    if scale is not None:
        s = np.abs(np.asarray(scale, np.float64))
        mag = mag * (s if scale_mode == 0 else 1.0 / s)[None, :]
    return mag


@pytest.mark.parametrize("q", [3, 4])
def test_legacy_one_sided_matches_reference(golden, q):
    import coset_amd
    V = golden("vlut_legacy")
    mgr = coset_amd.vLUTManager(coset_amd.LegacyE8Lattice(), coset_amd.QuantizationConfig(lattice_type="E8", q=q, M=2))
    for i in range(2):
        a = torch.from_numpy(V[f"q{q}_a{i}"])
        v = mgr.build_one_sided_vlut(a)
        assert v.device.type == "cpu" and v.shape == (q ** 8,)
        close(v.numpy(), V[f"q{q}_vlut{i}"], abs_residuals(q, True) @ np.abs(V[f"q{q}_a{i}"].astype(np.float64)),
              1e-6)
        assert mgr.build_one_sided_vlut(a) is v  # cached


def test_core_one_sided_matches_oracle():
    import coset_amd
    rng = np.random.default_rng(4)
    a = rng.standard_normal((3, 8)).astype(np.float32)
    for q in (2, 4):
        v = coset_amd.build_one_sided_vluts(torch.from_numpy(a), q, legacy=False).cpu().numpy()
        R = O.e8_decode(O.unpack_words(np.arange(q ** 8), q).reshape(-1, 1, 8), q, 1).astype(np.float64)
        for i in range(3):
            ref = R @ a[i].astype(np.float64)
            close(v[i], ref, np.abs(R) @ np.abs(a[i].astype(np.float64)), 1e-6)


def test_equal_sum_queries_get_their_own_tables():
    import coset_amd
    mgr = coset_amd.vLUTManager(coset_amd.LegacyE8Lattice(), coset_amd.QuantizationConfig(lattice_type="E8", q=3, M=2))
    a1 = torch.tensor([1., 0, 0, 0, 0, 0, 0, 0])
    a2 = torch.tensor([0., 1, 0, 0, 0, 0, 0, 0])
    assert not torch.equal(mgr.build_one_sided_vlut(a1), mgr.build_one_sided_vlut(a2))


def test_lookup_dot_equals_decode_then_dot():
    """tests/legacy/test_one_sided_vlut_pytest.py:294-333 on the core rule."""
    import coset_amd
    rng = np.random.default_rng(5)
    x = rng.standard_normal((500, 8)).astype(np.float32)
    a = rng.standard_normal(8).astype(np.float32)
    words = coset_amd.hnlq_encode(torch.from_numpy(x).cuda(), 4, 2, 1.0)
    vl = coset_amd.build_one_sided_vluts(torch.from_numpy(a).reshape(1, 8), 4, legacy=False)[0]
    got = coset_amd.vlut_dot(words, vl, 4).cpu().numpy()
    codes = O.e8_encode(x, 4, 2)
    dec = O.e8_decode(codes, 4, 2)
    words_np = O.pack_words(codes, 4).reshape(-1, 1, 2)
    mag = matmul_mag(words_np, 4, 2, a.reshape(1, 8))[0]
    close(got, dec.astype(np.float64) @ a.astype(np.float64), mag, 1e-6)


def test_reference_helpers():
    import coset_amd
    enc = torch.tensor([[1, 2, 3, 0, 0, 0, 0, 1]])
    assert int(coset_amd._encoding_to_index(enc, 4)[0]) == 4 ** 7 + 2 * 4 ** 6 + 3 * 4 ** 5 + 1
    mgr = coset_amd.vLUTManager(coset_amd.LegacyE8Lattice(), coset_amd.QuantizationConfig(lattice_type="E8", q=2, M=2))
    two = mgr.build_two_sided_vlut()
    pts = mgr._decode_encodings_to_lattice_points(mgr._generate_all_encodings()).double()
    torch.testing.assert_close(two.double(), pts @ pts.T)
    ex = [torch.randint(0, 2, (5, 8)) for _ in range(2)]
    ey = [torch.randint(0, 2, (5, 8)) for _ in range(2)]
    mac = coset_amd.vlut_mac_operation(ex, ey, two)
    ref = sum(two[coset_amd._encoding_to_index(ex[i], 2), coset_amd._encoding_to_index(ey[i], 2)] for i in range(2))
    torch.testing.assert_close(mac, ref)
    assert coset_amd.QuantizationConfig(lattice_type="E8", q=4, M=2).beta == 0.3


def runs(method, w):
    """Whether a weight form runs on a method: the pairs layout is read by
    the LDS-table method only."""
    return not (method == "mfma" and getattr(w, "layout", None) == "pairs")


@pytest.fixture(params=["bytes", "integer"])
def mfma_decode(request):
    """The MFMA kernel's two decoders: byte tables (default) and digits."""
    from coset_amd import _lib
    _lib.set_vlut_decode(request.param == "bytes")
    yield request.param
    _lib.set_vlut_decode(True)


@pytest.mark.parametrize("method", ["lds", "mfma"])
@pytest.mark.parametrize("B", [1, 3, 8, 17, 64, 80])
@pytest.mark.parametrize("adt", [torch.float16, torch.bfloat16, torch.float32])
def test_vlut_matmul_vs_oracle(method, B, adt, mfma_decode):
    import coset_amd
    if method == "lds" and mfma_decode == "integer":
        pytest.skip("decoder choice applies to the MFMA path")
    rng = np.random.default_rng(B)
    rows, K, q, M = 96, 320, 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(adt)
    for legacy in (False, True):
        prepared = [coset_amd.vlut_prepare(words, q, legacy=legacy, layout=lay)
                    for lay in ("rowmajor", "tiled", "pairs")]
        for mode in ("mul", "div"):
            sm = 0 if mode == "mul" else 1
            ref = O.vlut_matmul(words_np, scale, a.float().numpy(), q, M, scale_mode=sm, legacy=legacy)
            mag = matmul_mag(words_np, q, M, a.float().numpy(), scale, sm, legacy)
            for w in [words] + prepared:
                if not runs(method, w):
                    continue
                out = coset_amd.vlut_matmul(w, a.cuda(), q, scale=torch.from_numpy(scale), scale_mode=mode,
                                            legacy=legacy, method=method).cpu().numpy()
                close(out, ref, mag, RTOL[method])


@pytest.mark.parametrize("q,M", [(2, 1), (2, 2), (2, 3), (2, 4), (4, 1), (4, 3)])
@pytest.mark.parametrize("B", [1, 20])
def test_vlut_matmul_other_levels(q, M, B, mfma_decode):
    """q = 2 (byte decode up to M = 4) and q = 4 at M = 1 / 3 (M = 3 takes
    the integer decode): both methods against the oracle, raw and prepared
    words, core and legacy rules."""
    import coset_amd
    rng = np.random.default_rng(100 * q + 10 * M + B)
    rows, K = 80, 192
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(torch.float16)
    scale = np.ones(rows, np.float32)
    for legacy in (False, True):
        ref = O.vlut_matmul(words_np, scale, a.float().numpy(), q, M, scale_mode=0, legacy=legacy)
        mag = matmul_mag(words_np, q, M, a.float().numpy(), legacy=legacy)
        prepared = [coset_amd.vlut_prepare(words, q, legacy=legacy, layout=lay)
                    for lay in ("rowmajor", "tiled", "pairs")]
        for method in ("lds", "mfma"):
            for w in [words] + prepared:
                if not runs(method, w):
                    continue
                out = coset_amd.vlut_matmul(w, a.cuda(), q, legacy=legacy, method=method).cpu().numpy()
                close(out, ref, mag, RTOL[method])


@pytest.mark.parametrize("q,M", [(4, 2), (4, 1), (2, 3), (2, 4)])
@pytest.mark.parametrize("B", [1, 5, 11, 40])
def test_fp32_activations_on_matrix_cores(q, M, B):
    """fp32 activations on the MFMA method: each value split exactly into
    three bf16 planes (3B tokens), the planes' products summed per output;
    against the oracle's lookup sum (elementwise RTOL of the summands'
    magnitude), every weight format, both rules, with the bias + LSQ epilogue
    applied after the sum, and "auto" taking the same path."""
    import coset_amd
    rng = np.random.default_rng(7 * B + q + M)
    rows, K = 72, 136                        # 17 k-blocks
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    # magnitudes over 60 binades, so the low planes carry real bits
    a_np = (rng.standard_normal((B, K)) * np.exp2(rng.integers(-30, 30, (B, K)))).astype(np.float32)
    a = torch.from_numpy(a_np).cuda()
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    for legacy in (False, True):
        ref = O.vlut_matmul(words_np, scale, a_np, q, M, legacy=legacy)
        mag = matmul_mag(words_np, q, M, a_np, scale, 0, legacy)
        forms = [words] + [coset_amd.vlut_prepare(words, q, legacy=legacy, layout=lay)
                           for lay in ("rowmajor", "tiled", "decoded")]
        for w in forms:
            for method in ("mfma", "auto"):
                out = coset_amd.vlut_matmul(w, a, q, scale=torch.from_numpy(scale), legacy=legacy, method=method)
                close(out.cpu().numpy(), ref, mag, RTOL["mfma"])   # "auto" takes the matrix cores here
    # epilogue after the three planes' sum: bias, then the LSQ kernel's quantizer
    sc, bias = torch.from_numpy(scale).cuda(), torch.from_numpy(rng.standard_normal(rows).astype(np.float32)).cuda()
    m = coset_amd.LSQActivation(bit_width=6, init_alpha=3.0).cuda()
    plain = coset_amd.vlut_matmul(words, a, q, scale=sc, method="mfma")
    only_bias = coset_amd.vlut_matmul(words, a, q, scale=sc, bias=bias, method="mfma")
    fused = coset_amd.vlut_matmul(words, a, q, scale=sc, bias=bias, act_quant=(m.alpha, m.qmax), method="mfma")
    assert torch.equal(only_bias, plain + bias)
    with torch.no_grad():
        assert torch.equal(fused, m(plain + bias))


@pytest.mark.parametrize("n_tok", [6, 5])
def test_fp32_split_special_values(n_tok):
    """Infinities and NaN in fp32 activations reach the products whole (the
    planes after them hold 0): an output is finite exactly where the oracle's
    fp32 table sum is (which of NaN and +-inf a non-finite output takes can
    differ: the matrix-core method multiplies the decoded weight, the tables
    multiply each level's residual), a NaN activation makes its token's
    outputs NaN, and finite outputs agree with the oracle.  Five tokens take
    the rows kernel that splits the activations in its staging, six the
    separate split launch."""
    import coset_amd
    rng = np.random.default_rng(31)
    rows, K, q, M = 48, 64, 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a_np = rng.standard_normal((6, K)).astype(np.float32)
    a_np[1, 3] = np.inf
    a_np[2, 10] = -np.inf
    a_np[3, 20] = np.nan
    a_np[4, 5], a_np[4, 40] = np.inf, -np.inf
    a_np[5] *= np.float32(1e30)
    a_np = np.ascontiguousarray(a_np[:n_tok])
    ref = O.vlut_matmul(words_np, np.ones(rows, np.float32), a_np, q, M)
    out = coset_amd.vlut_matmul(words, torch.from_numpy(a_np).cuda(), q, method="mfma").cpu().numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(out), fin)
    assert np.isnan(out[3]).all() and not fin[1:5].any() and fin[0].all() and fin[5:].all()
    mag = matmul_mag(words_np, q, M, np.where(np.isfinite(a_np), a_np, 0))
    close(out[fin], ref[fin], mag[fin], RTOL["mfma"])


def _split3_np(a):
    """The exact three-plane split of finite fp32 values (h1 = a truncated to
    bf16, h2 = (a - h1) truncated, h3 = (a - h1 - h2) truncated), as uint16
    planes [3, ...]."""
    a = np.asarray(a, np.float32)
    hs, r = [], a
    for _ in range(3):
        h = (r.view(np.uint32) >> 16).astype(np.uint16)
        hs.append(h)
        r = (r - (h.astype(np.uint32) << 16).view(np.float32)).astype(np.float32)
    return np.stack(hs)


@pytest.mark.parametrize("B,rows,K", [(1, 80, 256), (8, 80, 256), (21, 64, 512), (40, 128, 4096), (40, 72, 136)])
def test_fp32_plane_sum_is_the_planes_products(B, rows, K):
    """The fp32 path adds each output's three plane products in the last
    kernel of its plan (the rows kernel, or the reduce of a split deep
    kernel; other plans through a separate sum): bit for bit
    ((y_1 + y_2) + y_3) + bias of the three bf16 planes run as 3B tokens of
    their own, for the raw words and the decoded format."""
    import coset_amd
    rng = np.random.default_rng(B * 1000 + rows + K)
    q, M = 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    words_np = O.pack_words(O.e8_encode(W.reshape(-1, 8), q, M), q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a_np = (rng.standard_normal((B, K)) * np.exp2(rng.integers(-20, 20, (B, K)))).astype(np.float32)
    planes = _split3_np(a_np).reshape(3 * B, K)
    p_bf = torch.from_numpy(planes.view(np.int16)).cuda().view(torch.bfloat16)
    sc = torch.from_numpy(rng.uniform(0.5, 2.0, rows).astype(np.float32)).cuda()
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float32)).cuda()
    for w in (words, coset_amd.vlut_prepare(words, q, layout="decoded")):
        y = coset_amd.vlut_matmul(w, p_bf, q, scale=sc, method="mfma")
        want = ((y[:B] + y[B:2 * B]) + y[2 * B:]) + bias
        got = coset_amd.vlut_matmul(w, torch.from_numpy(a_np).cuda(), q, scale=sc, bias=bias, method="mfma")
        assert torch.equal(got, want)


@pytest.mark.parametrize("deep", [1, 0])
@pytest.mark.parametrize("splits", [3, 8, 64])
@pytest.mark.parametrize("B,rows,K", [(40, 128, 4096), (40, 72, 136)])
def test_fp32_plane_sum_on_split_wide_and_deep_kernels(deep, splits, B, rows, K):
    """fp32 activations on a forced K split of the deep kernel and of the
    wide one (set_vlut_deep(False)): the split-major partials reach the fused
    three-plane reduce with the indexing each kernel writes, so the output is
    bit for bit ((y_1 + y_2) + y_3) + bias of the planes run as 3B tokens
    under the same plan."""
    import coset_amd
    from coset_amd import _lib
    rng = np.random.default_rng(B * 7 + rows + K + splits)
    q, M = 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    words_np = O.pack_words(O.e8_encode(W.reshape(-1, 8), q, M), q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a_np = (rng.standard_normal((B, K)) * np.exp2(rng.integers(-20, 20, (B, K)))).astype(np.float32)
    planes = _split3_np(a_np).reshape(3 * B, K)
    p_bf = torch.from_numpy(planes.view(np.int16)).cuda().view(torch.bfloat16)
    sc = torch.from_numpy(rng.uniform(0.5, 2.0, rows).astype(np.float32)).cuda()
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float32)).cuda()
    try:
        _lib.set_vlut_deep(bool(deep))
        _lib.set_vlut_splits(splits)
        for w in (words, coset_amd.vlut_prepare(words, q, layout="decoded")):
            y = coset_amd.vlut_matmul(w, p_bf, q, scale=sc, method="mfma")
            want = ((y[:B] + y[B:2 * B]) + y[2 * B:]) + bias
            got = coset_amd.vlut_matmul(w, torch.from_numpy(a_np).cuda(), q, scale=sc, bias=bias, method="mfma")
            assert torch.equal(got, want)
            ref = O.vlut_matmul(words_np, sc.cpu().numpy(), a_np, q, M) + bias.cpu().numpy()
            _close_elem(got.cpu().numpy(), ref,
                        matmul_mag(words_np, q, M, a_np, sc.cpu().numpy()) + np.abs(bias.cpu().numpy()))
    finally:
        _lib.set_vlut_splits(0)
        _lib.set_vlut_deep(True)


def test_fp32_mfma_needs_exact_operands():
    """q = 4, M = 3 decodes beyond what bf16 holds exactly: method "mfma"
    refuses fp32 activations there, "auto" takes the LDS-table method."""
    import coset_amd
    rng = np.random.default_rng(2)
    rows, K, q, M = 16, 32, 4, 3
    codes = O.e8_encode(rng.standard_normal((rows * K // 8, 8)).astype(np.float32), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a_np = rng.standard_normal((3, K)).astype(np.float32)
    with pytest.raises(Exception):
        coset_amd.vlut_matmul(words, torch.from_numpy(a_np).cuda(), q, method="mfma")
    out = coset_amd.vlut_matmul(words, torch.from_numpy(a_np).cuda(), q, method="auto").cpu().numpy()
    close(out, O.vlut_matmul(words_np, np.ones(rows, np.float32), a_np, q, M),
          matmul_mag(words_np, q, M, a_np), RTOL["auto"])


@pytest.mark.parametrize("splits", [1, 2, 5, 64])
def test_vlut_matmul_forced_splits(splits):
    """Any K split count (clamped to the method's range) gives the same
    product; workspace sizing follows the forced count."""
    import coset_amd
    from coset_amd import _lib
    rng = np.random.default_rng(splits)
    rows, K, q, M = 128, 1024, 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((4, K)).astype(np.float32)).to(torch.float16)
    ref = O.vlut_matmul(words_np, np.ones(rows, np.float32), a.float().numpy(), q, M)
    mag = matmul_mag(words_np, q, M, a.float().numpy())
    pairs = coset_amd.vlut_prepare(words, q, layout="pairs")
    _lib.set_vlut_splits(splits)
    try:
        for method, w in (("lds", words), ("lds", pairs), ("mfma", words)):
            out = coset_amd.vlut_matmul(w, a.cuda(), q, method=method).cpu().numpy()
            close(out, ref, mag, RTOL[method])
    finally:
        _lib.set_vlut_splits(0)


@pytest.mark.parametrize("B", [1, 2, 8, 9, 16])
@pytest.mark.parametrize("K,splits", [(4096, 0), (4608, 1), (4608, 3)])
def test_rows_kernel_staged_and_direct_activations(B, K, splits):
    """Batches of one 16-token tile take the rows kernel with activations
    staged in LDS (token bounds 1, 8, 16) when a wave's K range is at most
    16 k-quads, and loaded straight into the A operands otherwise (K = 4608
    in one split: 18 k-quads per wave); every weight format and both input
    types against the oracle."""
    import coset_amd
    from coset_amd import _lib
    rng = np.random.default_rng(2000 + B + K)
    rows, q, M = 48, 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    forms = [words] + [coset_amd.vlut_prepare(words, q, layout=lay) for lay in ("rowmajor", "tiled", "decoded")]
    _lib.set_vlut_splits(splits)
    try:
        for dt in (torch.float16, torch.bfloat16):
            a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(dt)
            ref = O.vlut_matmul(words_np, scale, a.float().numpy(), q, M)
            mag = matmul_mag(words_np, q, M, a.float().numpy(), scale)
            for w in forms:
                out = coset_amd.vlut_matmul(w, a.cuda(), q, scale=torch.from_numpy(scale), method="mfma")
                close(out.cpu().numpy(), ref, mag, RTOL["mfma"])
    finally:
        _lib.set_vlut_splits(0)


@pytest.mark.parametrize("B", [1, 5, 17, 40, 70])
def test_vlut_matmul_ragged_shapes(B, mfma_decode):
    """Rows and k-blocks that fill no tile (37 rows, 13 k-blocks), token
    counts across the 16 / 32 / 64-token tilings, every weight format."""
    import coset_amd
    rng = np.random.default_rng(1000 + B)
    rows, K, q, M = 37, 104, 4, 2
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32))
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    a16 = a.numpy().astype(np.float16).astype(np.float32)
    ref = O.vlut_matmul(words_np, scale, a16, q, M)
    mag = matmul_mag(words_np, q, M, a16, scale)
    forms = [words] + [coset_amd.vlut_prepare(words, q, layout=lay) for lay in ("rowmajor", "tiled", "pairs")]
    for w in forms:
        for method in ("lds", "mfma"):
            if not runs(method, w):
                continue
            out = coset_amd.vlut_matmul(w, a.half().cuda(), q, scale=torch.from_numpy(scale),
                                        method=method).cpu().numpy()
            close(out, ref, mag, RTOL[method])


@pytest.mark.parametrize("q,M", [(4, 2), (4, 4), (2, 3)])
@pytest.mark.parametrize("B", [1, 2, 4, 8, 11])
def test_pairs_layout(q, M, B):
    """The pairs layout: the LDS-table method with fp32 activations (the
    method "auto" takes for them) against the oracle for token counts of
    each token tiling, core and legacy rules; "auto" on the layout runs the
    LDS-table method, "mfma" refuses it; the layout's words are the pair ids
    the tables give every word."""
    import coset_amd
    rng = np.random.default_rng(300 + 10 * q + M + B)
    rows, K = 530, 264                   # two 512-row workgroups, a partial k-quad
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32))
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    for legacy in (False, True):
        pairs = coset_amd.vlut_prepare(words, q, legacy=legacy, layout="pairs")
        ref = O.vlut_matmul(words_np, scale, a.numpy(), q, M, scale_mode=1, legacy=legacy)
        mag = matmul_mag(words_np, q, M, a.numpy(), scale, 1, legacy)
        for method in ("auto", "lds"):
            out = coset_amd.vlut_matmul(pairs, a.cuda(), q, scale=torch.from_numpy(scale), scale_mode="div",
                                        legacy=legacy, method=method).cpu().numpy()
            close(out, ref, mag, RTOL[method])
        with pytest.raises(ValueError):
            coset_amd.vlut_matmul(pairs, a.half().cuda(), q, legacy=legacy, method="mfma")
    # every word's ids name pairs whose values are the word's residual; the
    # layout is [rows / 64][kb][M][64 rows]
    R = O.residual_table(q, legacy=False, strided=True)
    kb = K // 8
    ids = coset_amd.vlut_prepare(words, q, layout="pairs").data.cpu().numpy().astype(np.uint32)
    ids = ids.reshape(-1, kb, M, 64).transpose(0, 3, 1, 2).reshape(-1, kb, M)
    assert ids.shape[0] == -(-rows // 64) * 64
    ids = ids[:rows].reshape(-1)
    idx = words_np.astype(np.int64).reshape(-1)
    for p_ in range(4):
        pid = (ids >> (8 * p_)) & 0xff
        key = R[idx, 2 * p_] * 64 + R[idx, 2 * p_ + 1]      # the pair's value, as one number
        assert pid.max() < 72
        # one id per distinct value and one value per id
        pairs_seen = np.unique(np.stack([pid, key]), axis=1)
        assert len(np.unique(pairs_seen[0])) == pairs_seen.shape[1] == len(np.unique(pairs_seen[1]))


def _close_elem(out, ref, mag, rtol=1e-3):
    """Elementwise |out - ref| <= rtol * mag, mag = |a| @ |W|^T (>= |ref|)."""
    out, ref, mag = (np.asarray(t, np.float64) for t in (out, ref, mag))
    bad = np.abs(out - ref) > rtol * np.maximum(mag, np.abs(ref))
    assert not bad.any(), (int(bad.sum()), float(np.abs(out - ref)[bad].max()))


# Elementwise bounds of a C4 output, as fractions of its summands' magnitude
# |a| @ |W|^T.  Matrix cores: the fp16 x 2 x_hat products are exact and each
# output passes through at most 2^10 fp32 roundings (the MFMAs' sums over a
# wave's K range, the 8 waves' sum, the split reduce, the scale), each within
# 2^-24 of that magnitude.  LDS tables: the pair table entries are rounded
# products and an output sums up to 4096 of them in fp32.  A single wrong
# level-1 word moves an output by ~1e-3 of its magnitude at this size, far
# outside both.
C4_RTOL = {"mfma": 2.0 ** -14, "lds": 2.0 ** -12}


def test_c4_full_size_equals_decoded_product():
    """C4: 4096 x 4096 weights ~ N(0, 0.02) encoded with beta = 0.02 (q4 M2),
    fp16 activations at B = 1, 8, 64; every weight format and both methods
    against the oracle's lookup sum on 48 sampled rows and against
    a @ decode^T on all rows, elementwise within the summation-order bound
    of C4_RTOL."""
    import coset_amd
    g = torch.Generator(device="cuda").manual_seed(5)
    W = 0.02 * torch.randn((4096, 4096), device="cuda", generator=g)
    words = coset_amd.hnlq_encode(W.reshape(-1, 8), 4, 2, 0.02).reshape(4096, 512, 2)
    forms = {"words": words, "tiled": coset_amd.vlut_prepare(words, 4),
             "decoded": coset_amd.vlut_prepare(words, 4, layout="decoded"),
             "decoded6": coset_amd.vlut_prepare(words, 4, layout="decoded6"),
             "pairs": coset_amd.vlut_prepare(words, 4, layout="pairs")}
    dec = coset_amd.hnlq_decode(words.reshape(-1, 2), 4, 2, 0.02).reshape(4096, 4096)
    rows = np.arange(7, 4096, 85)
    words_rows = words.cpu().numpy().astype(np.uint32)[rows]
    for B in (1, 8, 64):
        a = torch.randn((B, 4096), device="cuda", generator=g).to(torch.float16)
        af = a.float().cpu().numpy()
        ref_rows = O.vlut_matmul(words_rows, np.full(len(rows), 0.02, np.float32), af, 4, 2)
        mag_rows = np.abs(af).astype(np.float64) @ np.abs(dec[rows].cpu().numpy().astype(np.float64)).T
        ref = (a.double() @ dec.double().T)
        mag = (a.double().abs() @ dec.double().abs().T)
        for method in ("lds", "mfma"):
            for name, w in forms.items():
                if (name.startswith("decoded") and method == "lds") or not runs(method, w):
                    continue
                print(f"C4 B={B} {method} {name}", flush=True)
                out = coset_amd.vlut_matmul(w, a, 4, scale=torch.full((4096,), 0.02), method=method)
                rtol = C4_RTOL[method]
                _close_elem(out[:, rows].cpu().numpy(), ref_rows, mag_rows, rtol)
                err = ((out.double() - ref).abs() / mag).max().item()
                print(f"  max |out - a decode^T| / magnitude = {err:.3g} (bound {rtol:.3g})", flush=True)
                assert err <= rtol, (B, method, name, err)


@pytest.mark.parametrize("deep", [1, 0])
@pytest.mark.parametrize("splits", [0, 1, 3, 8, 64])
@pytest.mark.parametrize("B", [33, 64, 100])
def test_wide_batch_kernels_vs_oracle(deep, splits, B):
    """Batches above 32 tokens (the deep kernel, or the wide one) with ragged
    rows and K, any forced K split, every weight format: against the
    oracle's lookup sum, elementwise within RTOL of |a| @ |W|^T."""
    import coset_amd as ca
    from coset_amd import _lib
    rng = np.random.default_rng(17 * B + splits)
    rows, K = 200, 1064                    # rows % 64 != 0, K / 8 = 133 k-blocks (not a multiple of 4)
    W = rng.standard_normal((rows, K)).astype(np.float32)
    codes = O.e8_encode(W.reshape(-1, 8), 4, 2)
    words_np = O.pack_words(codes, 4).reshape(rows, K // 8, 2)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(torch.bfloat16)
    af = a.float().numpy()
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    ref = O.vlut_matmul(words_np, scale, af, 4, 2)
    decw = O.e8_decode(codes, 4, 2).reshape(rows, K) * scale[:, None]
    mag = np.abs(af).astype(np.float64) @ np.abs(decw).T.astype(np.float64)
    forms = [words] + [ca.vlut_prepare(words, 4, layout=lay) for lay in ("rowmajor", "tiled", "decoded")]
    try:
        _lib.set_vlut_deep(bool(deep))
        _lib.set_vlut_splits(splits)
        outs = []
        for w in forms:
            out = ca.vlut_matmul(w, a.cuda(), 4, scale=torch.from_numpy(scale), method="mfma")
            _close_elem(out.cpu().numpy(), ref, mag, RTOL["mfma"])
            outs.append(out)
    finally:
        _lib.set_vlut_splits(0)
        _lib.set_vlut_deep(True)
    for o in outs[1:]:                     # the formats feed identical MFMA operands
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("q,M", [(4, 2), (4, 1), (2, 3), (2, 4)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 8, 40, 64])
def test_decoded_format_equals_tiled(q, M, dt, B):
    """Format 3 (2 x_hat bytes decoded once) feeds the same MFMA operands as
    the tiled cid|idx format, so the outputs are bit-equal; both equal the
    dense product with the decoded weights to fp32 summation order."""
    import coset_amd as ca
    torch.manual_seed(11 + B)
    rows, K = 72, 520                      # ragged: rows % 16 != 0, K/8 % 4 != 0
    x = torch.randn(rows * K // 8, 8, device="cuda") * 1.5
    words = ca.hnlq_encode(x, q, M, 1.0).reshape(rows, K // 8, M)
    tiled = ca.vlut_prepare(words, q, layout="tiled")
    dec = ca.vlut_prepare(words, q, layout="decoded")
    a = torch.randn(B, K, device="cuda").to(dt)
    scale = torch.rand(rows, device="cuda") + 0.5
    y2 = ca.vlut_matmul(tiled, a, scale=scale)
    y3 = ca.vlut_matmul(dec, a, scale=scale)
    assert torch.equal(y2, y3)
    W = ca.hnlq_decode(words.reshape(-1, M), q, M, None).reshape(rows, K) * scale.view(-1, 1)
    ref = a.float() @ W.t()
    mag = a.float().abs() @ W.abs().t()
    assert ((y3 - ref).abs() <= RTOL["mfma"] * mag).all()


def _unpack_decoded6(data, rows, kb):
    """Host decoder of the 6-byte format (include/coset_amd.h, format 5):
    returns 2 x_hat [rows, kb, 8] (int) and the field offset it implies is
    checked by the caller."""
    kq = -(-kb // 4)
    chunks = -(-kq // 8)
    w = data.cpu().numpy().astype(np.uint32).reshape(-(-rows // 16), chunks, 64, 12)
    bits = np.zeros(w.shape[:3] + (384,), np.uint8)
    for i in range(12):
        for b in range(32):
            bits[..., 32 * i + b] = (w[..., i] >> b) & 1
    out = np.zeros((rows, kb, 8), np.int64)
    for rt in range(w.shape[0]):
        for ch in range(chunks):
            for lane in range(64):
                row = rt * 16 + (lane & 15)
                for st in range(8):
                    k = (ch * 8 + st) * 4 + (lane >> 4)
                    if row >= rows or k >= kb:
                        continue
                    v = bits[rt, ch, lane, 48 * st:48 * st + 48].astype(np.int64)
                    byte = [int(np.dot(v[8 * i:8 * i + 8], 1 << np.arange(8))) for i in range(6)]
                    top = [b_ >> 6 for b_ in byte]
                    f = [b_ & 63 for b_ in byte]
                    f.append(top[0] | top[1] << 2 | top[2] << 4)
                    v7 = top[3] | top[4] << 2 | top[5] << 4
                    f.append(v7 & 31)
                    p = v7 >> 5
                    out[row, k] = [2 * (fj - 18) + p for fj in f]
    return out


@pytest.mark.parametrize("legacy", [False, True])
def test_decoded6_format_holds_the_decode(legacy):
    """Format 5 read back on the host: every pair's 2 x_hat equals the
    oracle's decode of its two level words (q = 4, M = 2, offset 18), on a
    ragged shape whose padding the reader skips."""
    import coset_amd as ca
    rng = np.random.default_rng(61 + legacy)
    rows, K, q, M = 40, 328, 4, 2                  # kb = 41: a partial chunk
    codes = O.e8_encode((rng.standard_normal((rows * K // 8, 8)) * 2).astype(np.float32), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    d6 = ca.vlut_prepare(words, q, legacy=legacy, layout="decoded6")
    got = _unpack_decoded6(d6.data, rows, K // 8)
    R = O.residual_table(q, legacy=legacy, strided=True).reshape(-1, 8)
    want = np.zeros((rows, K // 8, 8), np.int64)
    for m in range(M):
        want += (q ** m) * np.rint(2 * R[words_np[:, :, m].astype(np.int64)]).astype(np.int64)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("q,M", [(4, 2), (4, 1)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 5, 8, 16, 17, 33, 40, 64, 100])
@pytest.mark.parametrize("splits", [0, 3])
def test_decoded6_matmul_vs_oracle(q, M, dt, B, splits):
    """Format 5 on the rows (B <= 32) and deep (B > 32) kernels, ragged rows
    and K (partial chunks), natural and forced K splits: elementwise against
    the oracle's lookup sum within RTOL of the summands' magnitude, and within
    2^-16 of it against the 8-byte decoded format (the same exact operands,
    the waves' K ranges aligned to chunks)."""
    import coset_amd as ca
    from coset_amd import _lib
    rng = np.random.default_rng(100 * B + 10 * M + splits)
    rows, K = 200, 1064                            # rows % 16 != 0, kb = 133 (not a multiple of 32)
    codes = O.e8_encode(rng.standard_normal((rows * K // 8, 8)).astype(np.float32), q, M)
    words_np = O.pack_words(codes, q).reshape(rows, K // 8, M)
    words = torch.from_numpy(words_np.astype(np.int32)).to(torch.uint16).cuda()
    a = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(dt)
    af = a.float().numpy()
    scale = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    ref = O.vlut_matmul(words_np, scale, af, q, M)
    mag = matmul_mag(words_np, q, M, af, scale)
    d6 = ca.vlut_prepare(words, q, layout="decoded6")
    d8 = ca.vlut_prepare(words, q, layout="decoded")
    try:
        _lib.set_vlut_splits(splits)
        y6 = ca.vlut_matmul(d6, a.cuda(), q, scale=torch.from_numpy(scale), method="mfma")
        y8 = ca.vlut_matmul(d8, a.cuda(), q, scale=torch.from_numpy(scale), method="mfma")
    finally:
        _lib.set_vlut_splits(0)
    _close_elem(y6.cpu().numpy(), ref, mag, RTOL["mfma"])
    _close_elem(y6.cpu().numpy(), y8.cpu().numpy(), mag, 2.0 ** -16)


@pytest.mark.parametrize("B", [1, 8, 64])
def test_decoded6_bit_equal_to_decoded_at_4096(B):
    """At the C4 shape (4096 x 4096: one K split on the rows kernel, four on
    the deep kernel) every wave's K range is whole chunks under both formats,
    so the kernels see identical operands in identical order: the outputs
    are bit-equal (fp16 and fp32 activations).  (Where the planner splits K
    into ranges that are not whole chunks, the 6-byte format's waves take
    chunk-aligned ranges and the sums' order differs.)"""
    import coset_amd as ca
    g = torch.Generator(device="cuda").manual_seed(9)
    W = 0.02 * torch.randn((4096, 4096), device="cuda", generator=g)
    words = ca.hnlq_encode(W.reshape(-1, 8), 4, 2, 0.02).reshape(4096, 512, 2)
    d6, d8 = ca.vlut_prepare(words, 4, layout="decoded6"), ca.vlut_prepare(words, 4, layout="decoded")
    scale = torch.full((4096,), 0.02, device="cuda")
    for dt in (torch.float16, torch.float32):
        a = torch.randn((B, 4096), device="cuda", generator=g).to(dt)
        assert torch.equal(ca.vlut_matmul(d6, a, scale=scale, method="mfma"),
                           ca.vlut_matmul(d8, a, scale=scale, method="mfma")), (B, dt)


def test_decoded6_rejects_what_it_cannot_hold():
    import coset_amd as ca
    from coset_amd import _lib
    with pytest.raises(Exception):
        ca.vlut_prepare(torch.zeros(16, 4, 3, dtype=torch.uint16, device="cuda"), 4, layout="decoded6")
    d6 = ca.vlut_prepare(torch.zeros(16, 4, 2, dtype=torch.uint16, device="cuda"), 4, layout="decoded6")
    a = torch.randn(40, 32, device="cuda").half()
    with pytest.raises(Exception):
        ca.vlut_matmul(d6, a, method="lds")                # the LDS-table method reads no decoded bytes
    try:
        _lib.set_vlut_deep(False)                          # the wide kernel reads the 8-byte format only
        with pytest.raises(Exception):
            ca.vlut_matmul(d6, a, method="mfma")
    finally:
        _lib.set_vlut_deep(True)
    assert torch.equal(ca.vlut_matmul(d6, a), torch.zeros(40, 16, device="cuda"))


def test_decoded_format_rejects_what_it_cannot_hold():
    import coset_amd as ca
    words = torch.zeros(16, 4, 3, dtype=torch.uint16, device="cuda")
    with pytest.raises(Exception):
        ca.vlut_prepare(words, 4, layout="decoded")      # q = 4, M = 3 overflows a byte
    dec = ca.vlut_prepare(torch.zeros(16, 4, 2, dtype=torch.uint16, device="cuda"), 4, layout="decoded")
    a = torch.randn(2, 32, device="cuda")
    with pytest.raises(Exception):
        ca.vlut_matmul(dec, a, method="lds")                 # the LDS-table method reads no decoded bytes
    assert torch.equal(ca.vlut_matmul(dec, a), torch.zeros(2, 16, device="cuda"))   # fp32: the three-plane path
