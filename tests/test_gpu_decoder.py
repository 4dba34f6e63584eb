"""GPU: one Llama-style decoder layer (BASELINE C5's composition) forward and backward through
libhk.so against float64 torch autograd of the same layer on the CPU, with the layer's own BF16
parameters. The layer keeps BF16 activations (each rounding ~2^-9 relative), so the comparison is
normwise: ||a - b|| / ||b|| <= 1e-2 for the output and every gradient, a bound that a wiring
mistake (a missing residual, a transposed projection, an unrotated head) exceeds by far.

C5 itself (hidden 4096, 32/8 heads, FFN 14336, 2 x 2048 tokens) runs at full size on the GPU with
dY nonzero only on the first 128 positions of each sequence. Attention is causal, so those
positions' outputs and every gradient depend on the first 128 positions only (a later query's dO
is zero, so its dS row is zero and it adds nothing to dK, dV or any weight gradient): the float64
reference over 2 x 128 tokens with the same weights pins the full-size kernels exactly."""
import numpy as np
import pytest
import torch

from rust_ascend_hip import DecoderConfig, DecoderLayer
from rust_ascend_hip.decoder import rope_tables

pytestmark = pytest.mark.gpu

SMALL = DecoderConfig(hidden=256, heads=4, kv_heads=2, ffn=512, vocab=1000, batch=2, seq=128)
TOL = 1e-2


def reference(layer: DecoderLayer, ids, dy):
    """float64 autograd of the layer over ids [B, S'] (S' <= the layer's seq: a prefix of each
    sequence) with upstream dy [B*S', H]."""
    c = layer.cfg
    P = {k: getattr(layer, k).detach().double().cpu().requires_grad_(True)
         for k in ("table", "wqkv", "wo", "wg", "wu", "wd", "w1", "w2")}
    seq = ids.shape[1]
    T, H, D, hq, hkv = c.batch * seq, c.hidden, c.head_dim, c.heads, c.kv_heads
    cos, sin = (torch.from_numpy(t).double() for t in rope_tables(seq, D, c.theta))

    def rms(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + c.eps) * w

    def rope(x):  # x [B, H, S, D], split-half pairs
        a, b = x[..., :D // 2], x[..., D // 2:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], -1)

    x0 = P["table"][ids.reshape(-1)]
    n1 = rms(x0, P["w1"])
    qkv = (n1 @ P["wqkv"].T).reshape(c.batch, seq, hq + 2 * hkv, D).permute(0, 2, 1, 3)
    q, k, v = rope(qkv[:, :hq]), rope(qkv[:, hq:hq + hkv]), qkv[:, hq + hkv:]
    k, v = k.repeat_interleave(hq // hkv, 1), v.repeat_interleave(hq // hkv, 1)
    s = (q @ k.transpose(-1, -2)) * D ** -0.5
    s = s.masked_fill(torch.triu(torch.ones(seq, seq, dtype=torch.bool), 1), float("-inf"))
    o = (torch.softmax(s, -1) @ v).permute(0, 2, 1, 3).reshape(T, H)
    h1 = x0 + o @ P["wo"].T
    n2 = rms(h1, P["w2"])
    m = torch.nn.functional.silu(n2 @ P["wg"].T) * (n2 @ P["wu"].T)
    y = h1 + m @ P["wd"].T
    (y * dy).sum().backward()
    return y.detach(), {k: t.grad for k, t in P.items()}


def normwise(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_layer(layer: DecoderLayer, ids, dy, prefix: int):
    """Run the layer on the GPU and compare the first `prefix` positions of each sequence (dy must
    be zero after them) and every parameter gradient with the float64 reference."""
    c = layer.cfg
    y = layer.forward(ids)[:, :prefix].float().cpu().numpy().reshape(c.batch * prefix, c.hidden)
    grads = {k: v.float().cpu().numpy() for k, v in layer.backward(dy).items()}
    y_ref, g_ref = reference(layer, ids[:, :prefix].cpu(),
                             dy[:, :prefix].double().cpu().reshape(c.batch * prefix, c.hidden))
    errors = {"y": normwise(y, y_ref.numpy())}
    used = np.unique(ids[:, :prefix].cpu().numpy())
    for k, ref in g_ref.items():
        ref = ref.numpy()
        got = grads[k]
        if k == "table":
            assert not np.any(np.delete(got, used, axis=0)), "rows of IDs without a gradient must stay zero"
            got, ref = got[used], ref[used]
        errors[k] = normwise(got, ref)
    print({k: f"{v:.2e}" for k, v in errors.items()}, flush=True)
    assert max(errors.values()) <= TOL, errors
    return grads


def test_decoder_layer_matches_float64_autograd():
    layer = DecoderLayer(SMALL, seed=3)
    c = SMALL
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    ids = torch.randint(0, c.vocab, (c.batch, c.seq), generator=g, device="cuda")
    ids[0, :10] = 5  # repeated IDs accumulate in the table gradient
    dy = torch.randn((c.batch, c.seq, c.hidden), generator=g, device="cuda").to(torch.bfloat16)
    grads = check_layer(layer, ids, dy, c.seq)
    # a second step on the same buffers reproduces the gradients bit for bit (deterministic)
    layer.forward(ids)
    again = layer.backward(dy)
    for k, v in again.items():
        assert np.array_equal(v.float().cpu().numpy(), grads[k]), k


def test_decoder_layer_c5_full_size_prefix_gradient():
    """BASELINE config C5 at full size (hidden 4096, 32/8 heads, FFN 14336, 2 x 2048 tokens,
    vocab 32000, N(0, 0.02) weights) with dY nonzero on the first 128 positions of each sequence."""
    c = DecoderConfig()
    prefix = 128
    layer = DecoderLayer(c, seed=5)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    ids = torch.randint(0, c.vocab, (c.batch, c.seq), generator=g, device="cuda")
    ids[1, 100:140] = ids[0, 3]  # an ID repeated inside and past the prefix
    dy = torch.randn((c.batch, c.seq, c.hidden), generator=g, device="cuda").to(torch.bfloat16)
    dy[:, prefix:] = 0
    check_layer(layer, ids, dy, prefix)
    del layer
    torch.cuda.empty_cache()


def test_decoder_layer_rejects_bad_config_and_ids():
    with pytest.raises(ValueError):
        DecoderLayer(DecoderConfig(hidden=256, heads=3, kv_heads=1, ffn=512, vocab=100, batch=1, seq=64))
    layer = DecoderLayer(SMALL)
    with pytest.raises(ValueError):
        layer.forward(torch.zeros((1, 7), dtype=torch.int64, device="cuda"))
