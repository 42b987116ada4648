"""srq_batch_decode_i4_noalloc (split-KV decode whose partial states live in
the library's fixed per-GPU scratch) against srq_batch_decode_i4 with a
caller workspace, both called through the C ABI: two calls in a row, the
second with a smaller input, each bit-identical to the workspace form (same
kernels, same chunk split) and within the decode tolerance of the float64
oracle attention; an input needing more than the scratch is refused."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.gpu_util import to_dev, to_np

pytestmark = pytest.mark.gpu
SCRATCH_BYTES = 8 << 20


def _cache(rng, B, T, H, page, L):
    indptr, indices, last = oa.page_table(B, T, page)
    pages = int(indices.max()) + 1
    data = rng.integers(0, 256, (pages, L, 2, H, page, 64)).astype(np.uint8)
    param = np.empty((pages, L, 2, H, page, 2), np.float16)
    param[..., 0] = rng.uniform(0.02, 0.3, param.shape[:-1])
    param[..., 1] = rng.uniform(-2.0, 2.0, param.shape[:-1])
    return data, param, indptr, indices, last


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _decode(lib, fn, o, q, dev, B, Hq, H, L, layer, page, chunks, tmp=None):
    args = [_ptr(o), _ptr(q)] + [_ptr(t) for t in dev] + [B, Hq, H, L, layer, page, 128]
    if fn == "srq_batch_decode_i4":
        args += [_ptr(tmp) if tmp is not None else None, chunks]
    else:
        args += [chunks]
    args.append(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return getattr(lib, fn)(*args)


@pytest.mark.parametrize("first,second", [
    ((8, 32, 8, 1000, 64, 8), (2, 8, 2, 300, 16, 4)),
    ((32, 32, 8, 4096, 256, 2), (1, 32, 8, 700, 256, 64)),
])
def test_noalloc_decode_matches_workspace_decode(first, second):
    from signrot_amd import _native
    lib = _native.lib()
    rng = np.random.default_rng(sum(first))
    L, layer = 2, 1
    for B, Hq, H, T, page, chunks in (first, second):   # the second call is smaller
        data, param, indptr, indices, last = _cache(rng, B, T, H, page, L)
        dev = [to_dev(a) for a in (data, param, indptr, indices, last)]
        q_np = rng.standard_normal((B, Hq, 128)).astype(np.float16)
        q = to_dev(q_np)
        o_ref = torch.empty_like(q)
        tmp = torch.empty((B, Hq, chunks, 132), dtype=torch.float32, device="cuda")
        assert B * Hq * chunks * 132 * 4 <= SCRATCH_BYTES
        rc = _decode(lib, "srq_batch_decode_i4", o_ref, q, dev, B, Hq, H, L, layer, page,
                     chunks, tmp)
        assert rc == 0, lib.srq_last_error()
        o = torch.full_like(q, float("nan"))
        rc = _decode(lib, "srq_batch_decode_i4_noalloc", o, q, dev, B, Hq, H, L, layer, page,
                     chunks)
        assert rc == 0, lib.srq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"B={B} chunks={chunks}: differs from the workspace form"
        want = oa.decode(q_np, data, param, indptr, indices, last, layer)
        got = to_np(o).astype(np.float64)
        assert np.all(np.abs(got - want) <= 1e-2 + 1e-2 * np.abs(want)), \
            f"B={B} chunks={chunks}: {np.abs(got - want).max()} from the oracle"


def test_noalloc_decode_refuses_more_than_the_scratch():
    from signrot_amd import _native
    lib = _native.lib()
    rng = np.random.default_rng(3)
    B, Hq, H, T, page, L = 64, 64, 8, 256, 64, 1
    data, param, indptr, indices, last = _cache(rng, B, T, H, page, L)
    dev = [to_dev(a) for a in (data, param, indptr, indices, last)]
    q = torch.zeros((B, Hq, 128), dtype=torch.float16, device="cuda")
    o = torch.zeros_like(q)
    chunks = 4          # 64 * 64 * 4 * 132 * 4 bytes = 8.25 MiB > 8 MiB
    rc = _decode(lib, "srq_batch_decode_i4_noalloc", o, q, dev, B, Hq, H, L, 0, page, chunks)
    assert rc != 0
    assert b"scratch" in lib.srq_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(o) == 0          # nothing was launched
    # one chunk needs no scratch at all
    rc = _decode(lib, "srq_batch_decode_i4_noalloc", o, q, dev, B, Hq, H, L, 0, page, 1)
    assert rc == 0, lib.srq_last_error()
