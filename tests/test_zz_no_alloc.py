"""bh_attention_noalloc, the allocation-free variant of bh_attention (its V^T and key-split
partials live in a fixed 64 MiB device array per GPU), through the C ABI against bh_attention on
the same operands: the same kernels and the same key splits, so the outputs are equal bit for bit.
Two calls in a row, the second smaller (the scratch keeps the first call's contents), a masked
call split over the keys, the head_dim-512 path, a head_dim with no scratch at all, and a call
whose V^T would not fit, which is refused before any launch."""
import numpy as np
import pytest

from helpers import BF16, F32

pytestmark = pytest.mark.gpu


def tensors(batch, heads, sq, skv, dh, seed, masked):
    import torch
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(batch, sq, heads * dh, device="cuda", generator=gen).bfloat16()
    k = torch.randn(batch, skv, heads * dh, device="cuda", generator=gen).bfloat16()
    v = torch.randn(batch, skv, heads * dh, device="cuda", generator=gen).bfloat16()
    mask = None
    if masked:
        mask = torch.zeros(batch, skv, device="cuda")
        for b in range(batch):
            mask[b, : max(1, (b + 1) * skv // 3)] = 1
    return q, k, v, mask


def both(batch, heads, sq, skv, dh, seed=0, masked=False):
    """(noalloc output, bh_attention output, free device bytes before and after the noalloc call)."""
    import torch
    import burnisher_amd as bh
    print(f"noalloc case B{batch} H{heads} Sq{sq} Skv{skv} d{dh} masked={masked}", flush=True)
    q, k, v, mask = tensors(batch, heads, sq, skv, dh, seed, masked)
    mp = None if mask is None else mask.data_ptr()
    a = torch.zeros_like(q)
    b = torch.zeros_like(q)
    call = lambda: bh.call("bh_attention_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(),
                           batch, heads, sq, skv, dh, 0.0, None, mp, F32, BF16, None)
    call()   # a kernel's first launch in a process may make the runtime set up its private memory
    torch.cuda.synchronize()
    first = a.clone()
    free0 = torch.cuda.mem_get_info()[0]
    call()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert torch.equal(a, first), "two identical calls differ"
    bh.call("bh_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), batch, heads, sq, skv,
            dh, 0.0, None, mp, F32, BF16, None)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    return a, b, free0, free1


def test_noalloc_equals_attention_two_calls_second_smaller(hip):
    import torch
    # 128 workgroups of 512 queries: both entry points split the keys in two (fp32 partials in
    # the scratch after V^T for the allocation-free one)
    a, b, f0, f1 = both(2, 16, 2048, 2048, 72, seed=1)
    assert torch.equal(a, b), "head_dim 72 self-attention differs from bh_attention"
    assert f1 == f0, f"the call changed free device memory by {f0 - f1} bytes"
    a, b, f0, f1 = both(1, 4, 300, 120, 72, seed=2, masked=True)
    assert torch.equal(a, b), "the second, smaller call differs from bh_attention"
    assert f1 == f0
    # and a third at the first size again: nothing left from the smaller call leaks in
    a, b, _, _ = both(2, 16, 2048, 2048, 72, seed=3)
    assert torch.equal(a, b)


def test_noalloc_key_split_masked(hip):
    import torch
    # 16 workgroups over 16 key blocks, a ragged last block and a caption-style mask: 8 key splits,
    # and the second batch row's mask leaves some splits with no live key
    a, b, f0, f1 = both(2, 4, 600, 1000, 72, seed=7, masked=True)
    assert torch.equal(a, b) and f1 == f0


def test_noalloc_head_dim_512_and_no_scratch_paths(hip):
    import torch
    a, b, f0, f1 = both(1, 1, 1024, 1024, 512, seed=4)
    assert torch.equal(a, b) and f1 == f0
    a, b, f0, f1 = both(2, 4, 77, 77, 64, seed=5, masked=True)   # the generic kernel: no V^T at all
    assert torch.equal(a, b) and f1 == f0


def test_noalloc_refuses_what_does_not_fit(hip):
    import torch
    import burnisher_amd as bh
    # V^T of 2 x 16 x 72 x 16384 bf16 = 75.5 MB > 64 MiB
    q, k, v, _ = tensors(2, 16, 64, 16384, 72, seed=6, masked=False)
    out = torch.zeros_like(q)
    with pytest.raises(bh.BurnisherError, match="above the fixed maximum"):
        bh.call("bh_attention_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 2, 16, 64,
                16384, 72, 0.0, None, None, F32, BF16, None)
    torch.cuda.synchronize()
    assert not out.any(), "a refused call wrote the output"
    host = np.zeros(16, np.uint16)
    with pytest.raises(bh.BurnisherError, match="HOST"):
        bh.call("bh_attention_noalloc", host.ctypes.data, k.data_ptr(), v.data_ptr(), out.data_ptr(), 1, 1,
                1, 1, 72, 0.0, None, None, F32, BF16, None)
