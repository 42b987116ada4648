"""Shared helpers for the GPU parity tests: seeded numpy inputs, device
transfer, and the first-mismatch report used in assertion messages."""
import numpy as np
import torch

DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def to_np(t):
    return t.detach().cpu().numpy()


def assert_bitexact(got, want, what):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype == np.float16:
        g, w = got.view(np.uint16), want.astype(np.float16).view(np.uint16)
    else:
        g, w = got, want
    bad = np.argwhere(g != w)
    assert bad.size == 0, (f"{what}: {len(bad)} / {g.size} differ; first at {tuple(bad[0])}: "
                           f"got {got[tuple(bad[0])]} want {want[tuple(bad[0])]}")


def outlier_input(rng, rows, cols, n_out=4, mag=100.0):
    """N(0,1) fp16 activations with a few seeded massive-outlier channels."""
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    ch = rng.permutation(cols)[:n_out]
    sg = rng.choice([-1.0, 1.0], n_out)
    x[:, ch] *= sg * mag
    return x.astype(np.float16)
