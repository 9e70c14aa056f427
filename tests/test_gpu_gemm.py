"""coset_gemm_tn: the weight gradient gy^T x of the layer's F.linear
(coset/core/layers.py:478, autograd's grad_weight), on the matrix cores.

Exactness pin: with small-integer bf16 operands every product and every
partial sum is an integer below 2^24, so the fp32 result is exact whatever
the summation order -- the kernel must equal the integer product bit for
bit (fp32 out) and its round-to-nearest-even (bf16 out).  A misplaced tile,
token or lane shows as a wrong integer.  Gaussian operands are checked
against an fp32 product at the fp32 accumulation bound.
"""
import numpy as np
import pytest
import torch

from coset_amd import _lib, layers

pytestmark = pytest.mark.gpu

# (M, N, K, tile): tile 0 is the plan's own choice, 64 or 96 forced
SHAPES = [
    (768, 768, 4096, 0),     # C5 768 -> 768: 144 tiles of 64 x 64, one split, XCD blocks 3 x 6
    (768, 768, 4096, 96),    # the same on 64 tiles of 96 x 96, 4 K splits and the ordered reduce
    (3072, 768, 4096, 0),    # C5 768 -> 3072: 256 tiles of 96 x 96, one split, XCD blocks 4 x 8
    (768, 3072, 4096, 0),    # C5 3072 -> 768: the transposed grid
    (512, 512, 4096, 0),     # 64 tiles of 64 x 64: 4 K splits
    (2048, 512, 2048, 0),    # 256 tiles, one split
    (1024, 1024, 1024, 0),   # 256 tiles, 4 slices per wave
    (64, 64, 8192, 0),       # one tile: 8 K splits
    (192, 320, 2048, 0),     # 15 tiles: no XCD blocks, 2 K splits
    (128, 64, 4096, 0),      # 2 tiles: 4 K splits
    (96, 96, 8192, 0),       # one 96 x 96 tile: 8 K splits
    (288, 480, 2048, 96),    # 15 tiles of 96 x 96: no XCD blocks, 2 K splits
]


@pytest.fixture
def tile():
    yield
    _lib.set_gemm_tn_tile(0)


def _workspace(M, N, K):
    need = int(_lib.load().coset_gemm_tn_workspace_floats(M, N, K))
    return torch.full((max(need, 4),), float("nan"), dtype=torch.float32, device="cuda"), need


def _tn(a, b, out_dtype, colsum=None):
    lib = _lib.load()
    K, M = a.shape
    N = b.shape[1]
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device="cuda")
    ws, need = _workspace(M, N, K)
    rc = lib.coset_gemm_tn(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), out.data_ptr(), out.stride(0),
                           _lib.BF16 if out_dtype == torch.bfloat16 else _lib.F32, M, N, K,
                           0 if colsum is None else colsum.data_ptr(), ws.data_ptr(), need, _lib.stream_of(a))
    _lib.check("coset_gemm_tn", rc)
    torch.cuda.synchronize()
    return out


def _int_operands(K, M, N, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randint(-4, 5, (K, M), device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randint(-4, 5, (K, N), device="cuda", generator=g).to(torch.bfloat16)
    exact = a.double().t() @ b.double()     # integers below 2^17: exact in fp32
    return a, b, exact


@pytest.mark.parametrize("M,N,K,T", SHAPES)
def test_integer_operands_exact(M, N, K, T, tile):
    print(f"gemm_tn exact M={M} N={N} K={K} tile={T}", flush=True)
    _lib.set_gemm_tn_tile(T)
    assert _lib.load().coset_gemm_tn_supported(M, N, K) == 1
    a, b, exact = _int_operands(K, M, N, seed=M + N + K)
    c32 = _tn(a, b, torch.float32)
    assert torch.equal(c32.double(), exact), "fp32 output differs from the exact integer product"
    cs = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
    c16 = _tn(a, b, torch.bfloat16, colsum=cs)
    assert torch.equal(c16, exact.float().to(torch.bfloat16)), "bf16 output is not the RNE of the exact product"
    # the column sums of A (the bias gradient when A = gy), exact integers too
    assert torch.equal(cs.double(), a.double().sum(0)), "column sums differ"


@pytest.mark.parametrize("M,N,K,T", [(768, 768, 4096, 0), (768, 768, 4096, 96), (512, 512, 4096, 0),
                                     (3072, 768, 4096, 0)])
def test_gaussian_operands_within_fp32_bound(M, N, K, T, tile):
    print(f"gemm_tn gaussian M={M} N={N} K={K} tile={T}", flush=True)
    _lib.set_gemm_tn_tile(T)
    g = torch.Generator(device="cuda").manual_seed(9)
    a = torch.randn((K, M), device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randn((K, N), device="cuda", generator=g).to(torch.bfloat16)
    ref = a.double().t() @ b.double()
    mag = a.double().abs().t() @ b.double().abs()
    c32 = _tn(a, b, torch.float32)
    # fp32 sums of K exact products: error below K * 2^-24 of the magnitude
    # in the worst case, ~sqrt(K) * 2^-24 typically; the bound is 2^-16
    assert ((c32.double() - ref).abs() <= 2.0 ** -16 * mag).all()
    c16 = _tn(a, b, torch.bfloat16)
    assert ((c16.double() - ref).abs() <= 2.0 ** -8 * ref.abs() + 2.0 ** -16 * mag).all()
    # deterministic: the same bits on every call
    assert torch.equal(_tn(a, b, torch.float32), c32)


def test_strided_operands():
    """Leading dimensions wider than the matrix (views into wider buffers)."""
    print("gemm_tn strided", flush=True)
    # one split; 4 splits and the reduce; 96 x 96 tiles with 2 splits
    for K, M, N in ((1024, 128, 192), (4096, 64, 128), (2048, 192, 288)):
        a_full, b_full, _ = _int_operands(K, M + 32, N + 64, seed=3)
        a, b = a_full[:, 16:16 + M], b_full[:, 8:8 + N]
        exact = a.double().t() @ b.double()
        lib = _lib.load()
        out = torch.full((M, N + 16), float("nan"), dtype=torch.float32, device="cuda")
        ws, need = _workspace(M, N, K)
        rc = lib.coset_gemm_tn(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), out.data_ptr(), out.stride(0),
                               _lib.F32, M, N, K, 0, ws.data_ptr(), need, _lib.stream_of(a))
        _lib.check("coset_gemm_tn", rc)
        torch.cuda.synchronize()
        assert torch.equal(out[:, :N].double(), exact)
        assert torch.isnan(out[:, N:]).all(), "wrote past the output columns"


def test_workspace_refusals(tile):
    """A split plan without (enough) workspace is refused before any launch."""
    lib = _lib.load()
    M, N, K = 512, 512, 4096
    need = int(lib.coset_gemm_tn_workspace_floats(M, N, K))
    assert need == 4 * (M * N + M)   # 64 tiles: four K splits (tiles' and column sums' partials)
    a = torch.zeros((K, M), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(need, dtype=torch.float32, device="cuda")
    for ptr, n in ((0, 0), (ws.data_ptr(), need - 1)):
        rc = lib.coset_gemm_tn(a.data_ptr(), M, a.data_ptr(), N, out.data_ptr(), N, _lib.BF16, M, N, K, 0, ptr, n,
                               _lib.stream_of(a))
        assert rc == -1, rc
    assert int(lib.coset_gemm_tn_workspace_floats(768, 768, 4096)) == 0     # 144 tiles of 64: no split
    assert int(lib.coset_gemm_tn_workspace_floats(3072, 768, 4096)) == 0    # 256 tiles of 96: no split
    _lib.set_gemm_tn_tile(96)
    assert int(lib.coset_gemm_tn_workspace_floats(768, 768, 4096)) == 4 * (768 * 768 + 768)   # 64 tiles of 96


def test_unsupported_shapes_refused(tile):
    lib = _lib.load()
    # not multiples of 64, K not 256 * 2^s * {4, 8, 16, 32}, more than 256
    # tiles of either size (the library GEMM takes those)
    for M, N, K in ((770, 768, 4096), (768, 768, 4000), (768, 10, 4096), (0, 768, 4096), (768, 768, 768),
                    (3072, 3072, 4096), (1536, 1920, 4096)):
        assert lib.coset_gemm_tn_supported(M, N, K) == 0, (M, N, K)
    # the 3072-wide C5 layers: 256 tiles of 96 x 96, 576 of 64 x 64
    assert lib.coset_gemm_tn_supported(3072, 768, 4096) == 1
    _lib.set_gemm_tn_tile(64)
    assert lib.coset_gemm_tn_supported(3072, 768, 4096) == 0
    _lib.set_gemm_tn_tile(96)
    assert lib.coset_gemm_tn_supported(512, 512, 4096) == 0
    a = torch.zeros((4000, 768), dtype=torch.bfloat16, device="cuda")
    assert layers.gemm_tn(a, a) is None


def test_layer_weight_grad_matches_torch():
    """The layer's weight and bias gradients through QATLinearFn, with the
    kernel on (bias gradient fused into its pass) and off (torch.mm and
    coset_colsum): dW within bf16 rounding, db within the fp32 sum bound."""
    print("gemm_tn layer weight grad", flush=True)
    torch.manual_seed(7)
    import coset_amd as ca
    layer = ca.create_e8_hnlq_linear(768, 768, q=4, M=2, Delta0=1.5)
    with torch.no_grad():
        layer.weight.normal_(0.0, 1.0)
    x = torch.randn(4096, 768, device="cuda").to(torch.bfloat16)
    gy = torch.randn(4096, 768, device="cuda").to(torch.bfloat16)
    grads = {}
    for on in (True, False):
        layers.set_gemm_tn(on)
        try:
            layer.zero_grad(set_to_none=True)
            y = layer(x)
            y.backward(gy)
            grads[on] = layer.weight.grad.clone()
            grads[(on, "b")] = layer.bias.grad.clone()
        finally:
            layers.set_gemm_tn(True)
    # the straight-through backward passes dW_q through (times the clamp
    # mask); both runs round an fp32 product to bf16, the two fp32 sums
    # differing by their accumulation error (a fraction of the summands'
    # magnitude |gy|^T |x|), so they agree to one bf16 rounding plus that
    d = (grads[True] - grads[False]).abs()
    mag = gy.float().abs().t() @ x.float().abs()
    assert (d <= 2.0 ** -7 * grads[False].abs() + 2.0 ** -16 * mag).all()
    assert (d == 0).float().mean() > 0.5, "most weights should see the same bf16 value"
    db_ref = gy.double().sum(0)
    bmag = gy.double().abs().sum(0)
    for on in (True, False):
        assert ((grads[(on, "b")].double() - db_ref).abs() <= 2.0 ** -16 * bmag).all()
