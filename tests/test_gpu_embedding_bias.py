"""GPU parity: the bias / residual add and its bias gradient, and the embedding lookup with its
dense weight gradient, through the C ABI against the oracle.

Bias add and the bias gradient are bit-exact (the reference's F32 order of
src/nn/affine.rs:21-25 and the pairwise column sum of runtime/normalization.rs:95-114), on the
reference's own cases of examples/bias_tensor.rs and on random data. The embedding lookup is a
copy (bit-exact); its gradient is compared with the float64 oracle at the reference's tolerance
1e-5 + 1e-5|b| (examples/embedding_tensor.rs:8) and must be deterministic.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_bf16, dev_f32, host
from rust_ascend_hip import HipRuntime, HkError, nn
from ref_cases import BIAS_SHAPES, bias_inputs, embedding_reference_inputs

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ bias / residual add

@pytest.mark.parametrize("shape", BIAS_SHAPES)
def test_bias_add_reference_cases(shape):
    x, r, b, dy = bias_inputs(shape)
    for mode in range(3):
        xt = dev_f32(x).requires_grad_(True)
        rt = dev_f32(r).requires_grad_(True)
        bt = dev_f32(b).requires_grad_(True)
        if mode == 0:
            y, want = nn.bias_add(xt, bt), oracle.bias_add_f32(x, b)
        elif mode == 1:
            y, want = nn.residual_bias_add(xt, rt, bt), oracle.bias_add_f32(x, b, r)
        else:
            y, want = nn.residual_bias_add(xt, xt, bt), oracle.bias_add_f32(x, b, x)
        assert tuple(y.shape) == shape and y.dtype == torch.float32
        np.testing.assert_array_equal(host(y), want)
        ((y + y) * dev_f32(dy)).sum().backward()  # bias_tensor.rs:34-35
        factor = 4 if mode == 2 else 2
        np.testing.assert_array_equal(host(xt.grad), factor * dy)
        if mode == 1:
            np.testing.assert_array_equal(host(rt.grad), 2 * dy)
        np.testing.assert_array_equal(host(bt.grad), oracle.bias_add_backward(2 * dy))
    # a fixed bias needs no gradient reduction (bias_tensor.rs:43-47)
    xt = dev_f32(x).requires_grad_(True)
    (nn.bias_add(xt, dev_f32(b)) * dev_f32(dy)).sum().backward()
    np.testing.assert_array_equal(host(xt.grad), dy)


def test_bias_add_order_and_nonfinite():
    one = np.ones(1, np.float32)
    y = HipRuntime.bias_add(dev_f32(1e20 * one), dev_f32(one), dev_f32(-1e20 * one))
    assert host(y)[0] == 1.0  # (1e20 + -1e20) + 1 (bias_tensor.rs:60-61)
    data = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1.0, -1.0], np.float32)
    y = host(HipRuntime.bias_add(dev_f32(data), dev_f32(np.ones(7, np.float32))))
    np.testing.assert_array_equal(y, data + np.float32(1))
    np.testing.assert_array_equal(np.signbit(y), np.signbit(data + np.float32(1)))


@pytest.mark.parametrize("rows,width", [(1, 64), (2, 7), (3, 33), (4096, 4096), (333, 520), (17, 4097)])
def test_bias_add_random_f32_and_bf16(rows, width):
    x = oracle.normal((rows, width), seed=rows, stream=80)
    r = oracle.normal((rows, width), seed=rows, stream=81)
    b = oracle.normal((width,), seed=rows, stream=82)
    np.testing.assert_array_equal(host(HipRuntime.bias_add(dev_f32(x), dev_f32(b), dev_f32(r))),
                                  oracle.bias_add_f32(x, b, r))
    np.testing.assert_array_equal(host(HipRuntime.bias_add(dev_f32(x), dev_f32(b))), oracle.bias_add_f32(x, b))
    xb, rb = oracle.bf16_round(x), oracle.bf16_round(r)
    y = HipRuntime.bias_add(dev_bf16(x), dev_f32(b), dev_bf16(r))
    assert y.dtype == torch.bfloat16
    # F32 arithmetic on the widened values, one BF16 rounding of the result
    np.testing.assert_array_equal(host(y), oracle.bf16_round(oracle.bias_add_f32(xb, b, rb)))


@pytest.mark.parametrize("rows", [0, 1, 2, 3, 5, 31, 32, 33, 100, 1025, 4103, 16384])
@pytest.mark.parametrize("width", [1, 7, 64, 4097])
def test_bias_add_backward_bit_exact(rows, width):
    if rows * width > 1 << 24:
        pytest.skip("bounded host time")
    dy = oracle.normal((rows, width), seed=rows * 7 + width, stream=83, std=3.0)
    got = host(HipRuntime.bias_add_backward(dev_f32(dy)))
    np.testing.assert_array_equal(got, oracle.bias_add_backward(dy) if rows else np.zeros(width, np.float32))


def test_bias_add_backward_order_and_rank():
    parts = np.array([[1e8], [-1e8], [1.0], [1.0]], np.float32)
    assert host(HipRuntime.bias_add_backward(dev_f32(parts)))[0] == 0.0  # the halving order
    parts5 = np.array([[1e8], [1.0], [-1e8], [1.0], [0.0]], np.float32)
    assert host(HipRuntime.bias_add_backward(dev_f32(parts5)))[0] == 2.0
    dy = oracle.normal((2, 3, 5, 9), seed=1, stream=84)
    np.testing.assert_array_equal(host(HipRuntime.bias_add_backward(dev_f32(dy))), oracle.bias_add_backward(dy))


def test_bias_add_rejects_bad_inputs():
    x = torch.zeros((4, 8), device=DEV)
    with pytest.raises(HkError):
        HipRuntime.bias_add(x, torch.zeros(7, device=DEV))
    with pytest.raises(HkError):
        HipRuntime.bias_add(x, torch.zeros(8, device=DEV), torch.zeros((4, 7), device=DEV))
    with pytest.raises(HkError):
        HipRuntime.bias_add(x.half(), torch.zeros(8, device=DEV))
    with pytest.raises(HkError):
        HipRuntime.bias_add(x, torch.zeros(8, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HkError):
        HipRuntime.bias_add_backward(x.to(torch.bfloat16))
    with pytest.raises(HkError):
        HipRuntime.bias_add(torch.zeros((4, 0), device=DEV), torch.zeros(0, device=DEV))  # width must be positive


# ------------------------------------------------------------------ embedding

@pytest.mark.parametrize("padding_idx", [None, 0])
@pytest.mark.parametrize("scale", [False, True])
def test_embedding_reference_cases(padding_idx, scale):
    weights, ids, upstream = embedding_reference_inputs()
    w = dev_f32(weights).requires_grad_(True)
    ids_t = torch.from_numpy(ids).to(DEV)
    y = nn.embedding(w, ids_t, padding_idx, scale)
    np.testing.assert_array_equal(host(y), oracle.embedding(weights, ids))
    dy = dev_f32(upstream)
    (y * dy + y * dy).sum().backward()  # embedding_tensor.rs:28
    close(host(w.grad), oracle.embedding_backward_f64(2 * upstream, ids, 7, padding_idx, scale), 1e-5, 1e-5, "dW")


def test_embedding_int64_rank1_and_empty():
    weights, _, _ = embedding_reference_inputs()
    ids = torch.tensor([2, 5], dtype=torch.int64, device=DEV)
    y = HipRuntime.embedding(dev_f32(weights), ids)
    assert tuple(y.shape) == (2, 65)
    np.testing.assert_array_equal(host(y), weights[[2, 5]])
    for shape in [(0, 3), (2, 0)]:  # embedding_tensor.rs:47-53
        w = dev_f32(weights).requires_grad_(True)
        out = nn.embedding(w, torch.zeros(shape, dtype=torch.int32, device=DEV))
        assert out.numel() == 0 and tuple(out.shape) == shape + (65,)
        out.sum().backward()
        np.testing.assert_array_equal(host(w.grad), np.zeros((7, 65), np.float32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("width", [4096, 65, 8])
def test_embedding_lookup_exact(dtype, width):
    vocab = 32000 if width == 4096 else 300
    table = torch.randn((vocab, width), device=DEV, dtype=torch.float32).to(dtype)
    ids = torch.randint(0, vocab, (2, 2048), device=DEV, dtype=torch.int64)
    out = HipRuntime.embedding(table, ids)
    assert out.dtype == dtype and tuple(out.shape) == (2, 2048, width)
    assert torch.equal(out, table[ids])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embedding_backward_c5_shape(dtype):
    """C5's embedding: 2 x 2048 IDs uniform in [0, 32000), H = 4096."""
    vocab, width = 32000, 4096
    rng = np.random.default_rng(11)
    ids = rng.integers(0, vocab, (2, 2048))
    ids[0, :64] = 7  # one heavily repeated ID
    g = oracle.normal((2, 2048, width), seed=2, stream=85)
    ids_t = torch.from_numpy(ids).to(DEV)
    if dtype == torch.float32:
        g32 = HipRuntime.embedding_backward(dev_f32(g), ids_t, vocab, padding_idx=3, scale_grad_by_freq=False)
        rows = np.unique(np.concatenate([ids.reshape(-1)[:600], [3, 7, 0, vocab - 1]]))
        want = oracle.embedding_backward_f64(g, ids, vocab, 3, False)
        close(host(g32[torch.from_numpy(rows).to(DEV)]), want[rows], 1e-5, 1e-5, "dW rows")
        assert int(torch.count_nonzero(g32).item()) == np.count_nonzero(want)  # untouched rows are zero
    else:
        gb = oracle.bf16_round(g)
        gbt = HipRuntime.embedding_backward(dev_bf16(g), ids_t, vocab, padding_idx=3)
        ref32 = HipRuntime.embedding_backward(dev_f32(gb), ids_t, vocab, padding_idx=3)
        # F32 accumulation of the widened rows, one BF16 rounding
        np.testing.assert_array_equal(host(gbt[:700]), oracle.bf16_round(host(ref32[:700])))


def test_embedding_backward_deterministic_and_repeated():
    vocab, width = 10, 256
    ids = torch.from_numpy(np.random.default_rng(5).integers(0, vocab, 8192)).to(DEV)
    ids[:4096] = 4  # a bucket of > 4096 positions
    g = torch.randn((8192, width), device=DEV)
    a = HipRuntime.embedding_backward(g, ids, vocab, scale_grad_by_freq=True)
    b = HipRuntime.embedding_backward(g, ids, vocab, scale_grad_by_freq=True)
    assert torch.equal(a, b)
    want = oracle.embedding_backward_f64(host(g), ids.cpu().numpy(), vocab, None, True)
    close(host(a), want, 1e-5, 1e-4, "repeated IDs")


def position_order_sums_f32(g, ids, vocab):
    """dW in float32 with every row summed in increasing position order (what the kernel's
    grouping promises), evaluated on the host one position at a time."""
    ids = np.asarray(ids).reshape(-1)
    g = np.asarray(g, np.float32).reshape(ids.size, -1)
    dw = np.zeros((vocab, g.shape[1]), np.float32)
    order = np.argsort(ids, kind="stable")  # positions of each ID, in increasing order
    bounds = np.searchsorted(ids[order], np.arange(vocab + 1))
    for v in np.unique(ids):
        acc = np.zeros(g.shape[1], np.float32)
        for p in order[bounds[v]:bounds[v + 1]]:
            acc = acc + g[p]
        dw[v] = acc
    return dw


@pytest.mark.parametrize("tokens,vocab", [(70000, 5000), (20000, (1 << 20) + 3), (4097, 40000), (1, 1),
                                          (8192, 32000), (8193, 32000), (3000, (1 << 20) + 3)])
def test_embedding_backward_groups_in_position_order(tokens, vocab):
    """The grouping by ID is a stable radix sort (8-bit digits): 70000 positions span 18 sort
    tiles and a two-level scan of the digit histograms; a 2^20 + 3 row table needs three digit
    passes (the result lands in the other buffer pair); 40001 count entries take a multi-tile
    scan; up to 8192 positions the sort runs in one workgroup's LDS (8192 and 3000 positions,
    the latter over three passes), 8193 takes the multi-workgroup kernels. Gradient rows are F32 with magnitudes spread over 2^-20 .. 2^20, so the F32 sum of a row
    depends on the order of its positions: the result must equal, bit for bit, the sums taken in
    increasing position order."""
    rng = np.random.default_rng(tokens + vocab)
    hot = rng.integers(0, vocab, 16)
    ids = np.where(rng.random(tokens) < 0.5, hot[rng.integers(0, 16, tokens)], rng.integers(0, vocab, tokens))
    width = 64
    g = (rng.standard_normal((tokens, width)) * np.exp2(rng.integers(-20, 21, (tokens, 1)))).astype(np.float32)
    ids_t = torch.from_numpy(ids.astype(np.int64)).to(DEV)
    print(f"embedding backward grouping: {tokens} positions, {vocab} rows", flush=True)
    dw = HipRuntime.embedding_backward(dev_f32(g), ids_t, vocab)
    used = np.unique(ids)
    want = position_order_sums_f32(g, ids, vocab)
    got = dw[torch.from_numpy(used).to(DEV)].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.int32), want[used].view(np.int32))
    assert int(torch.count_nonzero(dw).item()) == np.count_nonzero(want)
    again = HipRuntime.embedding_backward(dev_f32(g), ids_t, vocab)
    assert torch.equal(dw, again)


def test_embedding_out_of_range_ids_error_and_recover():
    weights, _, _ = embedding_reference_inputs()
    w = dev_f32(weights)
    for bad in ([1, 7], [-1, 2]):
        with pytest.raises(HkError):
            HipRuntime.embedding(w, torch.tensor(bad, dtype=torch.int32, device=DEV))
        with pytest.raises(HkError):
            HipRuntime.embedding_backward(torch.ones((2, 65), device=DEV),
                                          torch.tensor(bad, dtype=torch.int64, device=DEV), 7)
    # the context is not poisoned
    np.testing.assert_array_equal(host(HipRuntime.embedding(w, torch.tensor([6], dtype=torch.int32, device=DEV))),
                                  weights[[6]])


def test_embedding_rejects_bad_inputs():
    w = torch.zeros((7, 16), device=DEV)
    ids = torch.zeros((2, 3), dtype=torch.int32, device=DEV)
    with pytest.raises(HkError):
        HipRuntime.embedding(w, ids.float())                      # floating IDs
    with pytest.raises(HkError):
        HipRuntime.embedding(w.reshape(7, 4, 4), ids)             # rank-3 table
    with pytest.raises(HkError):
        HipRuntime.embedding(torch.zeros((0, 16), device=DEV), ids)  # nonempty IDs need rows
    with pytest.raises(HkError):
        HipRuntime.embedding(w, torch.zeros((1,) * 8, dtype=torch.int32, device=DEV))  # ID rank 8
    with pytest.raises(HkError):
        HipRuntime.embedding_backward(torch.zeros((2, 3, 16), device=DEV), ids, 7, padding_idx=7)
    with pytest.raises(HkError):
        HipRuntime.embedding_backward(torch.zeros((2, 4, 16), device=DEV), ids, 7)  # shape mismatch
    with pytest.raises(ValueError):
        nn.embedding(w, ids, padding_idx=9)
