"""The allocation-free attention entry point (run with -m gpu).

nb_attention_step_static runs the kernel of nb_attention_step with its split
partials and head counters in the library's static device array instead of
a caller workspace.  Called through the C ABI twice in a row -- the second
call on a smaller problem (fewer heads, a narrower head, a shorter
context), so it reads an array the first call left full of its own partials
-- it must give exactly what nb_attention_step gives on the same inputs
(outputs and caches bit-identical: same kernel, same summation order), and
both must match the torch fp32 restatement of the reference's attention
(inference/generate_torch.py:72-106) within 1e-5.
"""
import ctypes

import pytest
import torch

from nativebit_amd import _lib
from nativebit_amd.model import precompute_rope
from oracle import decode_ref as R

pytestmark = pytest.mark.gpu


def P(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def state_tensor(dev, pos):
    st = _lib.DecodeState(0, pos, 0, 0, 0)
    t = torch.zeros(32, dtype=torch.uint8, device=dev)
    t[:24].copy_(torch.frombuffer(bytearray(bytes(st)), dtype=torch.uint8))
    return t


def rel(a, b):
    a = torch.as_tensor(a).double().reshape(-1).cpu()
    b = torch.as_tensor(b).double().reshape(-1).cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def torch_attention(qkv, kc, vc, pos, H, D, ctx):
    """One token with the cache (keys [H][ctx][D]), generate_torch.py:72-98."""
    C = H * D
    cos, sin = precompute_rope(D, ctx)
    q = R.rope(qkv[:C].reshape(1, H, 1, D), cos, sin, pos)[0, :, 0]
    k = R.rope(qkv[C:2 * C].reshape(1, H, 1, D), cos, sin, pos)[0, :, 0]
    kc, vc = kc.clone(), vc.clone()
    kc[:, pos] = k
    vc[:, pos] = qkv[2 * C:].reshape(H, D)
    att = (kc[:, :pos + 1] @ (q * D ** -0.5).unsqueeze(-1)).squeeze(-1)
    out = (torch.softmax(att, dim=-1).unsqueeze(1) @ vc[:, :pos + 1]).reshape(C)
    return out, kc, vc


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_static_attention_equals_workspace_entry(dev, out_dtype):
    lib = _lib.load()
    odt = _lib.NB_F32 if out_dtype == torch.float32 else _lib.NB_BF16
    assert lib.nb_attention_static_scratch_bytes() <= 2 << 20
    # the second call is smaller in every dimension
    for H, D, ctx, pos in ((20, 128, 1024, 777), (4, 64, 96, 40)):
        print(f"[case] static attention H={H} D={D} ctx={ctx} pos={pos} {out_dtype}", flush=True)
        g = torch.Generator().manual_seed(H * 1000 + pos)
        kc = torch.randn(H, ctx, D, generator=g)
        vc = torch.randn(H, ctx, D, generator=g)
        qkv = torch.randn(3 * H * D, generator=g)
        cos, sin = precompute_rope(D, ctx)
        cosd, sind, qkvd = cos.to(dev), sin.to(dev), qkv.to(dev)
        st = state_tensor(dev, pos)
        # workspace entry point
        ka, va = kc.transpose(1, 2).contiguous().to(dev), vc.to(dev)
        work = torch.zeros(int(lib.nb_attention_work_floats(H)), device=dev)
        done = torch.zeros(H, dtype=torch.int32, device=dev)
        out_a = torch.empty(H * D, dtype=out_dtype, device=dev)
        _lib.check(lib.nb_attention_step(P(qkvd), P(ka), P(va), P(cosd), P(sind), P(st),
                                         P(work), P(done), P(out_a), odt, H, D, ctx, stream()))
        # allocation-free entry point, same inputs
        kb, vb = kc.transpose(1, 2).contiguous().to(dev), vc.to(dev)
        out_b = torch.full((H * D,), float("nan"), dtype=out_dtype, device=dev)
        _lib.check(lib.nb_attention_step_static(P(qkvd), P(kb), P(vb), P(cosd), P(sind), P(st),
                                                P(out_b), odt, H, D, ctx, stream()))
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b)
        assert torch.equal(ka, kb) and torch.equal(va, vb)
        ref, kr, vr = torch_attention(qkv, kc, vc, pos, H, D, ctx)
        tol = 1e-5 if out_dtype == torch.float32 else 4e-3
        assert rel(out_b.float(), ref) <= tol, rel(out_b.float(), ref)
        assert torch.allclose(kb.cpu().transpose(1, 2), kr, rtol=1e-6, atol=1e-6)
        assert torch.equal(vb.cpu(), vr)
