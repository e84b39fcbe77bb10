"""The allocation-free attention entry point (``svoo_vbsa_fused_fwd_noalloc``) against the workspace one
(``svoo_vbsa_fused_fwd``), both called through the C ABI: the same bits on two calls in a row, the second
smaller than the first (the static scratch keeps the first call's plan, which must not leak into the
second), and on a head whose sizes do not sum to S (NaN rows and the status flag on both)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _case(r, dev, h, qn, kn, s, density):
    def sizes(c):
        cuts = np.sort(r.integers(0, s + 1, size=(h, c - 1)), axis=1)
        z = np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1)
        return np.diff(z, axis=1).astype(np.int32)

    qs = torch.from_numpy(sizes(qn)).to(dev)
    ks = torch.from_numpy(sizes(kn)).to(dev)
    m = torch.from_numpy(r.random((h, qn, kn)) < density).to(dev)
    m[0, 0, :] = False  # an empty row
    qi = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(dev)
    ki = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(dev)
    q, k, v = (torch.from_numpy(r.standard_normal((h, s, 128)).astype(np.float32)).to(torch.bfloat16).to(dev)
               for _ in range(3))
    return dict(h=h, qn=qn, kn=kn, s=s, q=q, k=k, v=v, qi=qi, ki=ki, m=m, qs=qs, ks=ks)


def _run(c, noalloc):
    from svoo_amd import _lib

    h, s, qn, kn = c["h"], c["s"], c["qn"], c["kn"]
    dev = c["q"].device
    out = torch.full((1, s, h * 128), 7.0, dtype=torch.bfloat16, device=dev)  # old contents must not survive
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    args = [c["q"].data_ptr(), c["k"].data_ptr(), c["v"].data_ptr(), c["qi"].data_ptr(), c["ki"].data_ptr(),
            c["m"].data_ptr(), c["qs"].data_ptr(), c["ks"].data_ptr(), out.data_ptr(), h, h, s, 128, qn, kn]
    st = _lib.stream_of(dev)
    if noalloc:
        _lib.call("svoo_vbsa_fused_fwd_noalloc", *args, status.data_ptr(), st)
    else:
        L = _lib.lib()
        ws = _lib.workspace(L.svoo_vbsa_workspace_size(h, s, qn, kn), dev)
        _lib.call("svoo_vbsa_fused_fwd", *args, ws.data_ptr(), ws.numel(), status.data_ptr(), st)
    torch.cuda.synchronize()
    return out, int(status.item())


def test_noalloc_equals_workspace_entry_two_calls(gpu):
    r = np.random.default_rng(2024)
    big = _case(r, gpu, 4, 40, 300, 6000, 0.2)
    small = _case(r, gpu, 2, 7, 50, 900, 0.5)
    for name, c in (("first call (4 heads, S=6000)", big), ("second call, smaller (2 heads, S=900)", small)):
        say("noalloc vs workspace entry,", name)
        ref, st_ref = _run(c, noalloc=False)
        got, st = _run(c, noalloc=True)
        assert st_ref == 0 and st == 0
        assert torch.equal(got, ref)
        assert not torch.isnan(got).any()


def test_noalloc_flags_inconsistent_sizes_like_workspace_entry(gpu):
    r = np.random.default_rng(7)
    c = _case(r, gpu, 3, 9, 30, 1200, 0.4)
    c["ks"][1, 0] += 5  # head 1's key sizes no longer sum to S
    say("noalloc vs workspace entry, inconsistent sizes in head 1")
    ref, st_ref = _run(c, noalloc=False)
    got, st = _run(c, noalloc=True)
    assert st_ref == 1 and st == 1
    o = got.view(c["s"], c["h"], 128)
    assert torch.isnan(o[:, 1]).all()  # every row of the bad head is NaN
    assert not torch.isnan(o[:, 0]).any() and not torch.isnan(o[:, 2]).any()
    assert torch.equal(torch.nan_to_num(got, nan=0.0), torch.nan_to_num(ref, nan=0.0))
