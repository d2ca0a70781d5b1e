"""The allocation-free attention entry point (q4nx_gqa_decode_static) against q4nx_gqa_decode
with a caller's workspace: bit-identical outputs on two calls in a row (the second smaller),
on both attention kernels, and a refusal before any launch when the split records would not
fit the library's static scratch."""

import ctypes as C

import numpy as np
import pytest
import torch

from llmnputest_amd import _lib, ops

pytestmark = pytest.mark.gpu

HQ, HKV, D = 40, 8, 64
ERR_WS = -3
SCRATCH = 65536 + (8 << 20)   # Q4NX_STATIC_SCRATCH_BYTES


def _inputs(batch, lmax, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dev = torch.device("cuda:0")
    q = torch.randn((batch, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn((batch, HKV, lmax, D), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((batch, HKV, lmax, D), generator=g, device=dev).to(torch.bfloat16)
    lens = torch.tensor([lmax - 7 * i for i in range(batch)], dtype=torch.int32, device=dev)
    return q, kc, vc, lens


def _static(q, kc, vc, lens, n_split, pol):
    b = q.shape[0]
    out = torch.full((b, HQ, D), -1, dtype=torch.int16, device=q.device).view(torch.bfloat16)
    of = torch.full((b, HQ, D), float("nan"), dtype=torch.float32, device=q.device)
    rc = _lib.lib().q4nx_gqa_decode_static(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), of.data_ptr(), b, HQ, HKV,
        D, lens.data_ptr(), kc.shape[2], kc.stride(0), kc.stride(1), C.c_float(0.125),
        n_split, C.byref(pol), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc, out, of


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


@pytest.mark.parametrize("attn_mfma", [1, 0])
def test_static_scratch_matches_workspace_entry(attn_mfma):
    pol = ops.Policy(attn_mfma=attn_mfma)
    ws = ops.Workspace(ops.WS_COUNTER_BYTES + (16 << 20), device=torch.device("cuda:0"))
    # two calls in a row, the second on a smaller problem (fewer sequences and positions)
    for batch, lmax, seed in ((8, 4096, 1), (1, 700, 2)):
        print(f"case: attn_mfma={attn_mfma} batch={batch} L={lmax}", flush=True)
        q, kc, vc, lens = _inputs(batch, lmax, seed)
        ns = ops.gqa_decode_splits(batch, HQ, HKV, lmax, policy=pol)
        assert ns > 1                                      # the split records are used
        assert 65536 + batch * HKV * ns * (HQ // HKV) * 68 * 4 <= SCRATCH
        ref, ref32 = ops.gqa_decode(q, kc, vc, lens, 0.125, n_split=0, want_f32=True, ws=ws,
                                    policy=pol)
        rc, out, of = _static(q, kc, vc, lens, 0, pol)
        torch.cuda.synchronize()
        assert rc == 0, _lib.lib().q4nx_last_error().decode()
        assert torch.equal(_bits(out), _bits(ref))
        assert torch.equal(_bits(of), _bits(ref32))
        assert torch.isfinite(ref32).all()


def test_static_scratch_refuses_oversize():
    pol = ops.Policy()
    q, kc, vc, lens = _inputs(8, 1024, 3)
    n_split = 128   # 8 sequences x 8 kv heads x 128 splits x 5 heads x 272 B = 11 MB of records
    rc, out, of = _static(q, kc, vc, lens, n_split, pol)
    torch.cuda.synchronize()
    assert rc == ERR_WS
    assert "static scratch" in _lib.lib().q4nx_last_error().decode()
    assert torch.isnan(of).all() and (out.view(torch.int16) == -1).all()   # nothing launched
    # the scratch is still usable afterwards
    rc, out, of = _static(q, kc, vc, lens, 8, pol)
    ref, ref32 = ops.gqa_decode(q, kc, vc, lens, 0.125, n_split=8, want_f32=True, policy=pol)
    torch.cuda.synchronize()
    assert rc == 0, _lib.lib().q4nx_last_error().decode()
    assert torch.equal(_bits(of), _bits(ref32)) and torch.equal(_bits(out), _bits(ref))
    assert np.isfinite(of.cpu().numpy()).all()
