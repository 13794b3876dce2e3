"""The allocation-free attention forward (siq_attn_varlen_fwd_noalloc) against
the workspace entry point (siq_attn_varlen_fwd), through the C ABI.

It keeps its plan in a static device array shared by every call on a GPU:
two calls in a row (the second smaller, so stale plan entries of the first
must not leak into it) must each give bitwise the workspace path's output,
and sizes beyond the array are rejected before anything is launched.
"""

import pytest
import torch

from siq_vl_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _noalloc():
    return _lib.lib().siq_attn_varlen_fwd_noalloc


def _inputs(lengths, hq, hkv, d, seed):
    g = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    mk = lambda h: torch.randn(t, h, d, generator=g).to(torch.bfloat16).to(DEV)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return mk(hq), mk(hkv), mk(hkv), torch.tensor(cu, dtype=torch.int32, device=DEV)


def _strides(q, k, v, o):
    return _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                             o.stride(0), o.stride(1)])


def _with_workspace(q, k, v, cu, causal):
    L = _lib.lib()
    total, hq, d = q.shape
    hkv = k.shape[1]
    batch = cu.numel() - 1
    out = torch.empty_like(q)
    lse = torch.empty((hq, total), dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L.siq_attn_fwd_workspace_bytes(batch, total, k.shape[0], hq, hkv, d), 16),
                     dtype=torch.uint8, device=DEV)
    rc = L.siq_attn_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                               cu.data_ptr(), cu.data_ptr(), batch, 0, 0, total, k.shape[0], hq, hkv, d,
                               _strides(q, k, v, out), d**-0.5, int(causal), ws.data_ptr(), ws.numel(),
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "siq_attn_varlen_fwd")
    return out, lse


def _no_alloc(q, k, v, cu, causal, out=None, lse=None):
    total, hq, d = q.shape
    hkv = k.shape[1]
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty((hq, total), dtype=torch.float32, device=DEV) if lse is None else lse
    rc = _noalloc()(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), cu.data_ptr(),
                    cu.data_ptr(), cu.numel() - 1, 0, 0, total, k.shape[0], hq, hkv, d, _strides(q, k, v, out),
                    d**-0.5, int(causal), torch.cuda.current_stream().cuda_stream)
    return rc, out, lse


def test_two_calls_in_a_row_match_the_workspace_path():
    cases = [
        ([300, 17, 1000, 1, 129, 640], 12, 2, 128, True),   # first call: larger plan
        ([64, 5, 200], 16, 16, 64, False),                  # second call: fewer tiles, other heads
    ]
    for i, (lengths, hq, hkv, d, causal) in enumerate(cases):
        print(f"noalloc call {i}: lengths={lengths} hq={hq} hkv={hkv} d={d} causal={causal}", flush=True)
        q, k, v, cu = _inputs(lengths, hq, hkv, d, seed=i)
        ref_out, ref_lse = _with_workspace(q, k, v, cu, causal)
        rc, out, lse = _no_alloc(q, k, v, cu, causal)
        assert rc == 0, _lib.lib().siq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
        assert torch.equal(lse, ref_lse)


def test_sizes_beyond_the_static_scratch_are_rejected():
    # 70000 sequences need more than the 1 MiB plan array: refused before any launch
    q = torch.zeros(8, 12, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(8, 2, 128, dtype=torch.bfloat16, device=DEV)
    cu = torch.zeros(70001, dtype=torch.int32, device=DEV)
    out = torch.full_like(q, 3.0)
    lse = torch.full((12, 8), 3.0, device=DEV)
    fn = _noalloc()
    rc = fn(q.data_ptr(), k.data_ptr(), k.data_ptr(), out.data_ptr(), lse.data_ptr(), cu.data_ptr(), cu.data_ptr(),
            70000, 0, 0, 8, 8, 12, 2, 128, _strides(q, k, k, out), 0.1, 1, None)
    assert rc == _lib.SIQ_ERR_WORKSPACE
    assert b"static scratch" in _lib.lib().siq_last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()) and bool((lse == 3.0).all())
