"""GPU tests of the LM head's projection with the sampling prologue in its
epilogue (lmrs_lm_head_fwd): logits against the oracle's linear_kernel
(kernels/ffi/tensor_ffi.cu:230-258), within the bound a different f32
summation order allows, and the fused tile maxima identical to the same
statistic computed from the logits the kernel wrote."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TILE = 64


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from lmrs_amd import sampling as S

    S.lib()


def _dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _keys(bits):
    b = bits.astype(np.uint32)
    return np.where(b & 0x8000, ~b & 0xFFFF, b | 0x8000).astype(np.uint64)


def standalone_tile_max(y_bits):
    """Per row and 64-column tile: key << 32 | ~column of the largest logit in
    the total order, ties to the lower column (numpy, from the logits)."""
    rows, V = y_bits.shape
    nt = (V + TILE - 1) // TILE
    cols = np.arange(V, dtype=np.uint64)
    ent = (_keys(y_bits) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - cols)[None, :]
    pad = np.zeros((rows, nt * TILE), np.uint64)
    pad[:, :V] = ent
    return pad.reshape(rows, nt, TILE).max(axis=2)


def _check_against_oracle(xb, wb, y, tm, name):
    import oracle as O
    from lmrs_amd import workloads as W

    ref, acc, sa = O.linear_bf16(xb, wb)
    got = W.bf16_bits_to_f32(y).astype(np.float64)
    K = xb.shape[1]
    # the kernel's f32 sum differs from the sequential one by at most
    # 2 K 2^-24 sum |x w|; bf16 rounding adds half an ulp (2^-9 relative)
    tol = 2 * K * 2.0 ** -24 * sa + np.abs(acc.astype(np.float64)) * 2.0 ** -8 + 1e-30
    err = np.abs(got - acc.astype(np.float64))
    assert np.all(err <= tol), (name, float(np.max(err / tol)))
    same = float(np.mean(y == ref))
    print(f"[lm_head] {name}: bitwise equal to linear_kernel on {100 * same:.3f}% of logits", flush=True)
    assert same > 0.97, (name, same)
    assert np.array_equal(tm.view(np.uint64), standalone_tile_max(y)), name


@pytest.mark.parametrize("rows,K,V", [(1, 8, 1), (7, 64, 100), (64, 520, 4113), (300, 256, 700), (256, 1024, 2048)])
def test_lm_head_matches_the_oracle(rows, K, V):
    from lmrs_amd import sampling as S
    from lmrs_amd import workloads as W

    rng = np.random.default_rng(rows * 1000 + K + V)
    xb = W.f32_to_bf16_bits(rng.normal(0, 1, (rows, K)).astype(np.float32))
    wb = W.f32_to_bf16_bits((rng.normal(0, 1, (V, K)) / np.sqrt(K)).astype(np.float32))
    print(f"[case] lm_head rows={rows} K={K} V={V}", flush=True)
    y, tm = S.lm_head(_dev_bf16(xb), _dev_bf16(wb))
    torch.cuda.synchronize()
    _check_against_oracle(xb, wb, y.view(torch.int16).cpu().numpy().view(np.uint16), tm.cpu().numpy(),
                          f"{rows}x{K}x{V}")


def test_lm_head_special_values_and_ties():
    """Rows of equal logits (ties to the lowest column per tile), +-inf and NaN
    products, and all-negative rows: the tile maxima follow the total order."""
    from lmrs_amd import sampling as S
    from lmrs_amd import workloads as W

    rows, K, V = 6, 16, 200
    x = np.zeros((rows, K), np.float32)
    x[:, 0] = 1.0
    w = np.zeros((V, K), np.float32)
    w[:, 0] = 1.0                        # row 0: all logits 1 (ties)
    w[17, 0] = np.inf
    w[150, 0] = -np.inf
    x[1, 0] = -1.0                       # row 1: all -1, -inf at 17, +inf at 150
    x[2, 0], x[2, 1] = 1.0, np.inf       # row 2: w[:,1] = 0 gives inf * 0 = NaN
    x[3, 0] = 0.0                        # row 3: all zeros (0 * inf = NaN at 17 and 150)
    x[4, 0] = -2.0
    x[5, 0] = 3.0
    xb, wb = W.f32_to_bf16_bits(x), W.f32_to_bf16_bits(w)
    y, tm = S.lm_head(_dev_bf16(xb), _dev_bf16(wb))
    torch.cuda.synchronize()
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    import oracle as O

    ref, _, _ = O.linear_bf16(xb, wb)
    nan = (ref & 0x7FFF) > 0x7F80
    assert np.array_equal(np.where(nan, 0x7FFF, yb), np.where(nan, 0x7FFF, ref))
    assert np.array_equal(tm.cpu().numpy().view(np.uint64), standalone_tile_max(yb))


def test_lm_head_with_no_hidden_features_writes_zeros():
    """in_features = 0 through the C-ABI (non-null operand pointers, as a C
    caller may pass): no operand is read, every logit is +0 and each tile's
    maximum is its lowest column, ties going to the lower column."""
    import ctypes

    from lmrs_amd import sampling as S

    rows, V = 3, 130
    nt = (V + TILE - 1) // TILE
    dummy_x = torch.zeros(8, dtype=torch.bfloat16, device="cuda")
    dummy_w = torch.zeros(8, dtype=torch.bfloat16, device="cuda")
    out = torch.full((rows, V), 7.0, dtype=torch.bfloat16, device="cuda")
    tm = torch.zeros((rows, nt), dtype=torch.int64, device="cuda")
    s = torch.cuda.current_stream()
    print(f"[case] lm_head rows={rows} K=0 V={V}", flush=True)
    rc = S.lib().lmrs_lm_head_fwd(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(dummy_x.data_ptr()),
                                  ctypes.c_void_p(dummy_w.data_ptr()), rows, 0, V, S.DTYPE_BF16,
                                  ctypes.c_void_p(tm.data_ptr()), ctypes.c_void_p(s.cuda_stream))
    assert rc == S.LMRS_OK
    torch.cuda.synchronize()
    yb = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.all(yb == 0)
    expect = standalone_tile_max(yb)
    assert np.array_equal(tm.cpu().numpy().view(np.uint64), expect)
    assert np.all(np.uint64(0xFFFFFFFF) - (expect & np.uint64(0xFFFFFFFF)) == np.arange(nt, dtype=np.uint64) * TILE)


def test_lm_head_at_the_c3_shape_feeds_the_sampler():
    """rows 256, H 4096, V 128256 (C3's batch and vocab): the fused tile maxima
    equal the standalone statistic on the whole output, sampled logits lie
    within the summation bound of float64 dot products, and greedy sampling
    of the projected logits returns, per row, the column of the largest tile
    entry."""
    from lmrs_amd import sampling as S
    from lmrs_amd import workloads as W

    rows, K, V = 256, 4096, 128256
    rng = np.random.default_rng(77)
    xb = W.f32_to_bf16_bits(rng.normal(0, 1, (rows, K)).astype(np.float32))
    wb = W.f32_to_bf16_bits((rng.normal(0, 1, (V, K)) * (2.5 / np.sqrt(K))).astype(np.float32))
    print(f"[case] lm_head C3 shape rows={rows} K={K} V={V}", flush=True)
    y, tm = S.lm_head(_dev_bf16(xb), _dev_bf16(wb))
    out = S.sample_batch(y, top_k=[S.GREEDY] * rows)
    torch.cuda.synchronize()
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    tmn = tm.cpu().numpy().view(np.uint64)
    assert np.array_equal(tmn, standalone_tile_max(yb))
    best = tmn.max(axis=1)
    argmax = (np.uint64(0xFFFFFFFF) - (best & np.uint64(0xFFFFFFFF))).astype(np.int64)
    assert np.array_equal(out["token_ids"].cpu().numpy().astype(np.int64), argmax)
    # a sample of logits against float64 dot products
    xf, wf = W.bf16_bits_to_f32(xb).astype(np.float64), W.bf16_bits_to_f32(wb).astype(np.float64)
    rr = rng.integers(0, rows, 4000)
    cc = rng.integers(0, V, 4000)
    exact = np.einsum("ij,ij->i", xf[rr], wf[cc])
    sa = np.einsum("ij,ij->i", np.abs(xf[rr]), np.abs(wf[cc]))
    got = W.bf16_bits_to_f32(yb[rr, cc]).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2 * K * 2.0 ** -24 * sa + np.abs(exact) * 2.0 ** -8 + 1e-30)
