"""coset_vlut_matmul_noalloc (the vLUT matmul with its split-K partials in a
fixed per-device scratch array, for callers that cannot allocate) against
coset_vlut_matmul with a caller workspace: bit-equal outputs, on two calls
in a row with the second smaller, for each weight format; refusal of a plan
that needs more scratch than the array holds."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call_both(lib, _lib, wts, fmt, a, scale, rows, K, M=2, q=4, method=2):
    B = a.shape[0]
    dt = _lib.dtype_code(a.dtype)
    need = lib.coset_vlut_workspace_floats(B, rows, K, q, M, dt, method)
    ws = torch.empty(max(int(need), 1), dtype=torch.float32, device="cuda")
    ref = torch.full((B, rows), float("nan"), device="cuda")
    out = torch.full((B, rows), float("nan"), device="cuda")
    st = _lib.stream_of(a)
    _lib.check("coset_vlut_matmul", lib.coset_vlut_matmul(
        wts.data_ptr(), fmt, scale.data_ptr(), 0, a.data_ptr(), dt, B, rows, K, q, M, 0, method, ws.data_ptr(),
        ws.numel(), ref.data_ptr(), st))
    _lib.check("coset_vlut_matmul_noalloc", lib.coset_vlut_matmul_noalloc(
        wts.data_ptr(), fmt, scale.data_ptr(), 0, a.data_ptr(), dt, B, rows, K, q, M, 0, method, out.data_ptr(), st))
    torch.cuda.synchronize()
    return int(need), ref, out


@pytest.mark.parametrize("layout", ["words", "tiled", "decoded"])
def test_noalloc_matches_workspace_entry_point(layout):
    import coset_amd as ca
    from coset_amd import _lib
    _lib.require_gpu()                       # coset_init: tables and this device's scratch address
    lib = _lib.load()
    assert lib.coset_vlut_noalloc_scratch_floats() == 2 << 20
    torch.manual_seed(12)
    rows, K = 4096, 4096
    W = 0.02 * torch.randn(rows * K // 8, 8, device="cuda")
    words = ca.hnlq_encode(W, 4, 2, 0.02).reshape(rows, K // 8, 2)
    if layout == "words":
        wts, fmt = words, 0
    else:
        prep = ca.vlut_prepare(words, 4, layout=layout)
        wts, fmt = prep.data, prep.word_format
    scale = torch.full((rows,), 0.02, device="cuda")
    # first call: 64 tokens (split-K partials in the scratch), then a smaller one
    for B in (64, 5):
        print(f"noalloc layout={layout} B={B}", flush=True)
        a = torch.randn(B, K, device="cuda").to(torch.float16)
        need, ref, out = _call_both(lib, _lib, wts, fmt, a, scale, rows, K)
        assert torch.equal(out, ref), (layout, B)
        if B == 64:
            assert need > 0, "the first call should exercise the scratch"
    # ragged shape with a forced K split: the scratch is reused with another layout of partials
    try:
        _lib.set_vlut_splits(3)
        a = torch.randn(3, 520, device="cuda").to(torch.bfloat16)
        w2 = ca.hnlq_encode(torch.randn(40 * 65, 8, device="cuda"), 4, 2, 1.0).reshape(40, 65, 2)
        need, ref, out = _call_both(lib, _lib, w2, 0, a, torch.ones(40, device="cuda"), 40, 520)
        assert need > 0 and torch.equal(out, ref)
    finally:
        _lib.set_vlut_splits(0)


@pytest.mark.parametrize("layout", ["pairs", "tiled"])
def test_noalloc_lds_table_method(layout):
    """The LDS-table method (fp32 activations) through both entry points: its
    split-major partials in the scratch, then a smaller call."""
    import coset_amd as ca
    from coset_amd import _lib
    _lib.require_gpu()
    lib = _lib.load()
    torch.manual_seed(13)
    rows, K = 1024, 2048
    W = torch.randn(rows * K // 8, 8, device="cuda")
    words = ca.hnlq_encode(W, 4, 2, 1.0).reshape(rows, K // 8, 2)
    prep = ca.vlut_prepare(words, 4, layout=layout)
    scale = torch.rand(rows, device="cuda") + 0.5
    for B in (8, 3):
        print(f"noalloc lds layout={layout} B={B}", flush=True)
        a = torch.randn(B, K, device="cuda")
        need, ref, out = _call_both(lib, _lib, prep.data, prep.word_format, a, scale, rows, K, method=1)
        assert torch.equal(out, ref), (layout, B)
        assert need > 0, "a K split: the call exercises the scratch"


def test_noalloc_refuses_plans_beyond_its_scratch():
    from coset_amd import _lib
    _lib.require_gpu()
    lib = _lib.load()
    cap = lib.coset_vlut_noalloc_scratch_floats()
    # the matrix-core method at a large batch (the deep kernel, four K splits at
    # least) needs more partials than the array holds
    B, rows, K = 4096, 4096, 4096
    need = lib.coset_vlut_workspace_floats(B, rows, K, 4, 2, _lib.F16, 2)
    assert need > cap, need
    # buffers of the plan's real sizes (8 MiB words, 32 MiB fp16 activations,
    # 64 MiB fp32 output): should the size check ever regress, the call runs
    # in bounds and fails the return-code assert instead of faulting
    words = torch.zeros(rows, K // 8, 2, dtype=torch.uint16, device="cuda")
    act = torch.zeros(B, K, dtype=torch.float16, device="cuda")
    out = torch.empty(B, rows, dtype=torch.float32, device="cuda")
    rc = lib.coset_vlut_matmul_noalloc(words.data_ptr(), 0, None, 0, act.data_ptr(), _lib.F16, B, rows, K, 4, 2, 0,
                                       2, out.data_ptr(), _lib.stream_of(out))
    torch.cuda.synchronize()
    assert rc == _lib.EINVAL
    assert b"scratch" in lib.coset_last_error()
