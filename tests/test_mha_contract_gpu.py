"""The caller contract of the reference's MHA layer (mha.py:103-178) on the
HIP kernels: heads folded from [B, S, H*D] into the batch ([B*H, S, D]),
one sdpa call per training step, and the dropout offset advanced by
B*H*S_q*S_kv after each call (mha.py:162-165), so that consecutive calls
draw disjoint counter ranges.  Two calls are checked: their dropout masks,
read back through the production forward kernel, against the reference
predicate at each call's offset; that the second call's mask is the one a
single call over twice the batch would give its upper half (the counter is
linear, so the ranges are disjoint); and both calls' outputs and gradients,
unfolded back to [B, S, H*D], against the oracle."""
import numpy as np
import pytest
import torch

from _common import TOL, maxabs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def fold(x, H):
    """[B, S, H*D] -> [B*H, S, D] (split the feature axis, heads before sequence)."""
    B, S, F = x.shape
    return x.reshape(B, S, H, F // H).permute(0, 2, 1, 3).reshape(B * H, S, F // H).contiguous()


def unfold(x, B, H):
    """[B*H, S, D] -> [B, S, H*D]."""
    BH, S, D = x.shape
    return x.reshape(B, H, S, D).permute(0, 2, 1, 3).reshape(B, S, H * D)


def test_mha_two_training_calls(pkg, O):
    B, S, H, D, p, seed, off0 = 2, 256, 4, 64, 0.1, 11, 0
    scale = D ** -0.5
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    x = lambda: torch.randn((B, S, H * D), generator=g, device=DEV).to(torch.float16)
    offsets = [off0, off0 + B * H * S * S]  # the layer's offset before each call
    masks = []
    for call, off in enumerate(offsets):
        print(f"[case] mha call {call} offset {off}", flush=True)
        q, k, v, d_o = x(), x(), x(), x()
        q3, k3, v3, do3 = (fold(t, H) for t in (q, k, v, d_o))
        o3, s3 = pkg.sdpa(q3, k3, v3, seed, off, dropout=p, scale=scale, causal_mask=True)
        dq3, dk3, dv3 = pkg.sdpa_grad(q3, k3, v3, o3, s3, do3, seed, off, dropout=p, scale=scale,
                                      causal_mask=True)
        torch.cuda.synchronize()
        # outputs and gradients, compared in the caller's [B, S, H*D] layout
        n = lambda t: t.cpu().numpy()
        okw = dict(scale=scale, dropout=p, causal_mask=True, seed=seed, offset=off)
        o_ref, s_ref = O.sdpa_fwd_gate(n(q3), n(k3), n(v3), **okw)
        g_ref = O.sdpa_bwd_gate(n(q3), n(k3), n(v3), n(o3), n(s3), n(do3), **okw)
        assert maxabs(n(unfold(o3, B, H)), n(unfold(torch.from_numpy(o_ref), B, H))) <= TOL["f16"]["o"]
        assert maxabs(n(s3), s_ref) <= TOL["f16"]["stats"]
        for got, ref in zip((dq3, dk3, dv3), g_ref):
            assert maxabs(n(unfold(got, B, H)), n(unfold(torch.from_numpy(ref), B, H))) <= TOL["f16"]["grad"]
        # the call's dropout mask through the production forward: q = 0, one-hot V
        mask = np.zeros((B * H, S, S), np.uint8)
        zq = torch.zeros_like(q3)
        for t in range(S // D):
            sel = torch.zeros_like(v3)
            j = torch.arange(D * t, D * t + D, device=DEV)
            sel[:, j, j - D * t] = 1
            o_sel, _ = pkg.sdpa(zq, k3, sel, seed, off, dropout=p, scale=scale, causal_mask=True)
            mask[:, :, D * t:D * t + D] = (o_sel > 0).cpu().numpy()
        ref = O.keep_mask(B * H, S, S, p, seed, off) & np.tril(np.ones((S, S), np.uint8))[None]
        assert np.array_equal(mask, ref), (call, int((mask != ref).sum()))
        masks.append(mask)
    # disjoint counter ranges: call 2 draws what batches B*H .. 2*B*H - 1 of one
    # call over twice the batch would draw, not call 1's mask again
    both = O.keep_mask(2 * B * H, S, S, p, seed, off0) & np.tril(np.ones((S, S), np.uint8))[None]
    assert np.array_equal(masks[0], both[:B * H]) and np.array_equal(masks[1], both[B * H:])
    assert not np.array_equal(masks[0], masks[1])
