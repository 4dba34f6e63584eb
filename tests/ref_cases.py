"""Input formulas of the reference's own device examples, shared by the oracle and GPU tests."""
import numpy as np

BIAS_SHAPES = [(1,), (7,), (3, 31), (2, 3, 33), (5, 4097), (2, 0, 7), (1, 2, 1, 3, 1, 1, 1, 7)]


def bias_inputs(shape):
    """examples/bias_tensor.rs:13-17 (shapes :57-58): integer-formula X, residual, bias and dY."""
    width, count = shape[-1], int(np.prod(shape))
    i = np.arange(count)
    x = ((i % 13) / 8 - 0.5).astype(np.float32).reshape(shape)
    r = ((i % 5) / 4 - 0.25).astype(np.float32).reshape(shape)
    b = ((np.arange(width) % 7) / 16 - 0.125).astype(np.float32)
    dy = ((i % 11) / 8 - 0.375).astype(np.float32).reshape(shape)
    return x, r, b, dy


def embedding_reference_inputs():
    """examples/embedding_tensor.rs:20-24: V = 7, H = 65, repeated IDs, integer-formula values."""
    vocab, width = 7, 65
    weights = (np.arange(vocab * width) / 8 - 2).astype(np.float32).reshape(vocab, width)
    ids = np.array([2, 0, 2, 5, 0, 2], np.int32).reshape(2, 3)
    upstream = ((np.arange(ids.size * width) % 17) / 8 - 0.5).astype(np.float32).reshape(2, 3, width)
    return weights, ids, upstream
