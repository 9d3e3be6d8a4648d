"""esda_decode_noalloc (the allocation-free decode entry point) against esda_decode.

Both run the same plan and kernels, so on identical inputs their outputs and cache
bytes must be identical bit for bit.  Each GPU test makes two noalloc calls in a row,
the second with a smaller input, so the second reads a scratch array that still holds
the first call's partials and table.  The size refusal runs on the host only.
"""
import ctypes

import numpy as np
import pytest
import torch

from apertura_amd import _lib
from apertura_amd.decode import DecodeStep, decode_status, decode_step, decode_step_noalloc, new_workspace

SCRATCH_BYTES = 32 << 20


def _rows(gen, shape):
    """Unit-RMS bf16 rows drawn on the device (both paths read the same tensors, so no
    host copy or oracle is needed)."""
    x = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
    return (x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)


def _pair(name, *, B, Hq, Hkv, D, cap, pos, window=0, ring=False, shared=False, seed=0, status=None):
    """esda_decode and esda_decode_noalloc on copies of the same inputs; returns the
    noalloc output."""
    print(f"\n[case] noalloc {name}: B={B} Hq={Hq} Hkv={Hkv} D={D} cap={cap} window={window} "
          f"ring={ring} shared={shared}", flush=True)
    scale = D ** -0.5
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    dstep = DecodeStep(batch=B, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, cap=cap, window=window,
                       ring=ring, kv_shared=shared, scale=scale)
    q_d, kn_d = _rows(gen, (B, Hq, D)), _rows(gen, (B, Hkv, D))
    vn_d = None if shared else _rows(gen, (B, Hkv, D))
    kc = _rows(gen, (B, Hkv, cap, D))
    vc = kc if shared else _rows(gen, (B, Hkv, cap, D))
    pos_d = torch.tensor(list(pos), dtype=torch.int32, device="cuda")
    caches = [(kc, vc), (kc.clone(), None)]
    caches[1] = (caches[1][0], caches[1][0] if shared else vc.clone())
    # both outputs start equal: a skipped sequence's rows are left as they were
    ref = decode_step(dstep, q_d, kn_d, vn_d, caches[0][0], caches[0][1], pos_d,
                      out=torch.zeros_like(q_d), workspace=new_workspace(dstep, "cuda"))
    out = torch.zeros_like(q_d)
    decode_step_noalloc(dstep, q_d, kn_d, vn_d, caches[1][0], caches[1][1], pos_d, out, status=status)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"{name}: noalloc output differs from esda_decode"
    assert torch.equal(caches[1][0].view(torch.int16), caches[0][0].view(torch.int16)), f"{name}: K cache bytes differ"
    if not shared:
        assert torch.equal(caches[1][1].view(torch.int16), caches[0][1].view(torch.int16)), \
            f"{name}: V cache bytes differ"
    return out


@pytest.mark.gpu
def test_noalloc_grid_plans_two_calls():
    """C4's shape (a grid of 64 splits per kv head: 4.2 MB of partials), then C1's
    (16 splits, D=256, a window) over the partials the first call left."""
    _pair("c4-shape", B=1, Hq=32, Hkv=4, D=512, cap=131072, pos=[131071], shared=True, seed=4)
    _pair("c1-shape", B=1, Hq=16, Hkv=8, D=256, cap=1024, window=1024, pos=[1023], seed=1)


@pytest.mark.gpu
def test_noalloc_balanced_plans_two_calls():
    """C5's global-layer shape (balanced shares over 32 ragged sequences), then a
    three-sequence batch whose table and slots are a prefix of the first call's."""
    rng = np.random.default_rng(55)
    pos = [int(x) - 1 for x in rng.integers(1024, 32769, size=32)]
    _pair("c5-global", B=32, Hq=32, Hkv=4, D=512, cap=32768, pos=pos, shared=True, seed=55)
    _pair("balanced-small", B=3, Hq=16, Hkv=2, D=512, cap=3000, pos=[2999, 100, 40], shared=True, seed=56)


@pytest.mark.gpu
def test_noalloc_ring_then_status_word():
    """A packed ring plan (C5's local shape), then a smaller step with one sequence out of
    range, counted into the caller's status word and skipped."""
    rng = np.random.default_rng(5)
    pos = [int(x) for x in rng.integers(0, 32768, size=32)]
    _pair("c5-local", B=32, Hq=32, Hkv=16, D=256, cap=1024, window=1024, ring=True, pos=pos, seed=5)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    step = DecodeStep(batch=2, num_q_heads=8, num_kv_heads=2, head_dim=128, cap=32)
    _pair("skip", B=2, Hq=8, Hkv=2, D=128, cap=32, pos=[5, 40], seed=8, status=status)
    assert decode_status(step, status) == 1
    assert decode_status(step, status) == 0


def test_noalloc_refuses_steps_beyond_the_scratch_without_device():
    """A plan whose partials exceed the static scratch is refused before any device call."""
    from apertura_amd.decode import workspace_bytes
    step = DecodeStep(batch=1, num_q_heads=32, num_kv_heads=4, head_dim=512, cap=131072, kv_shared=True,
                      split_rows=64)
    assert workspace_bytes(step) > SCRATCH_BYTES
    d = step.desc()
    fake = 0x10000  # never dereferenced: validation fails first
    a = _lib.DecodeArgs(fake, fake, None, fake, fake, fake, None, fake, None, 0)
    L = _lib.lib()
    assert L.esda_decode_noalloc(ctypes.byref(d), ctypes.byref(a), None) == 4
    assert b"static scratch" in L.esda_last_error()
    a.out = None
    assert L.esda_decode_noalloc(ctypes.byref(d), ctypes.byref(a), None) == 1
