"""bz_gemv_noalloc, the allocation-free variant of bz_gemv, through the C ABI.

It must give bz_gemv's results bit for bit (same kernels, same launch plan)
with its static per-GPU scratch in place of the caller's workspace, on calls
in a row whose sizes shrink (the scratch keeps the previous call's contents),
and refuse a call whose workspace exceeds BZ_GEMV_SCRATCH_BYTES before
launching anything."""

from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import bz_oracle as O
from tests._util import f32

from breeze_amd import _lib as L
from breeze_amd import gemv as G

pytestmark = pytest.mark.gpu


def _desc(x, w, wfmt, n, sc0=None, epilogue=L.EPI_NONE, residual=None, out=None, path=0, slices=0):
    d = L.GemvDesc()
    d.abi_version = L.ABI_VERSION
    d.M, d.K = x.shape
    d.N = n
    d.group = 128
    d.wfmt = wfmt
    d.epilogue = epilogue
    d.out_dtype = L.DT_BF16
    d.residual_dtype = L.DT_BF16
    d.cfg_path, d.cfg_slices = path, slices
    d.eps = 1e-6
    d.x, d.ldx = x.data_ptr(), x.stride(0)
    d.w = w.data_ptr()
    d.sc0 = None if sc0 is None else sc0.data_ptr()
    if residual is not None:
        d.residual, d.ldr = residual.data_ptr(), residual.stride(0)
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    return d


def _both(x, w, wfmt, n, **kw):
    """(bz_gemv with a zero-filled workspace of its own, bz_gemv_noalloc,
    workspace bytes the call needs)."""
    lib = L.lib()
    n_out = n // 2 if kw.get("epilogue") == L.EPI_SILU_GATE else n
    ref = torch.empty(x.shape[0], n_out, device=x.device, dtype=torch.bfloat16)
    got = torch.full_like(ref, float("nan"))
    d = _desc(x, w, wfmt, n, out=ref, **kw)
    need = lib.bz_gemv_workspace(ctypes.byref(d))
    ws = torch.zeros(max(need, 16) // 4 + 4, dtype=torch.int32, device=x.device)
    d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    L.check(lib.bz_gemv(ctypes.byref(d), L.stream_of(x)), "bz_gemv")
    d2 = _desc(x, w, wfmt, n, out=got, **kw)
    L.check(lib.bz_gemv_noalloc(ctypes.byref(d2), L.stream_of(x)), "bz_gemv_noalloc")
    torch.cuda.synchronize()
    return ref, got, need


def _int4(n, k, seed):
    w, _, _ = O.synth(n, k, 1, seed=seed)
    packed, sz, _ = G.quantize_int4_device(torch.from_numpy(w).cuda(), 128, False, G.W_INT4_ZP)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    return packed, sz, O.dequant_int4_zp(q, O.scales_zeros(s, z), 128)


def _fp8(n, k, seed):
    w, _, _ = O.synth(n, k, 1, seed=seed)
    codes, scale = G.quantize_fp8_device(torch.from_numpy(w).cuda(), 1e-12)
    c, sc = O.quantize_fp8_linear(w)
    return codes.view(torch.uint8), scale, O.dequant_fp8(c, sc)


def _x(m, k, seed):
    return torch.randn(m, k, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).cuda()


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
def test_noalloc_matches_bz_gemv_on_shrinking_calls(fmt):
    """down K10240 N2560 at M = 16 then 6 (split-K tile path, workspace
    1.6 MB then 0.6 MB), then M = 1 (no workspace)."""
    N, K = 2560, 10240
    w, sc, w_eff = _int4(N, K, 5) if fmt == "int4" else _fp8(N, K, 6)
    wfmt = G.W_INT4_ZP if fmt == "int4" else G.W_FP8
    needs = []
    for m in (16, 6, 1):
        x = _x(m, K, m)
        ref, got, need = _both(x, w, wfmt, N, sc0=sc)
        needs.append(need)
        assert torch.equal(got, ref), m
        assert O.rel_err(f32(got), O.gemv_ref(x.float().cpu().numpy(), w_eff)) <= 1e-2, m
    assert needs[0] > needs[1] > 0 and needs[2] == 0


def test_noalloc_tiled_several_rows():
    """A tiled weight at M = 12 then 5 (the panel kernel, no workspace) and
    at M = 32 over K10240 (the split-K tile kernel, with the scratch):
    bz_gemv's result bit for bit."""
    for n, k, ms in ((2560, 2560, (12, 5)), (2560, 10240, (32,))):
        w, sc, w_eff = _int4(n, k, 7)
        t = G.pack_tiled(G.W_INT4_ZP, w, k, G.W_INT4_TILED, sc0=sc)
        for m in ms:
            x = _x(m, k, 20 + m)
            ref, got, need = _both(x, t, G.W_INT4_TILED, n)
            assert torch.equal(got, ref), (k, m)
            assert (need > 0) == (k == 10240), (k, m, need)
            assert O.rel_err(f32(got), O.gemv_ref(x.float().cpu().numpy(), w_eff)) <= 1e-2, (k, m)


def test_noalloc_forced_slices_with_residual():
    """Forced tile path with 4 K slices over K2560 N4096: no epilogue at
    M = 8 then 5, a residual epilogue at M = 12 then 7."""
    K, N = 2560, 4096
    w, sc, w_eff = _int4(N, K, 7)
    for m in (8, 5):
        x = _x(m, K, 10 + m)
        ref, got, need = _both(x, w, G.W_INT4_ZP, N, sc0=sc, path=4, slices=4)
        assert need > 0 and torch.equal(got, ref), m
        assert O.rel_err(f32(got), O.gemv_ref(x.float().cpu().numpy(), w_eff)) <= 1e-2
    for m in (12, 7):
        x = _x(m, K, 20 + m)
        res = _x(m, N, 30 + m)
        ref, got, need = _both(x, w, G.W_INT4_ZP, N, sc0=sc, epilogue=L.EPI_RESIDUAL, residual=res, path=4,
                               slices=4)
        assert need > 0 and torch.equal(got, ref), m
        want = O.gemv_ref(x.float().cpu().numpy(), w_eff, O.EPI_RES, res.float().cpu().numpy())
        assert O.rel_err(f32(got), want) <= 1e-2


def test_noalloc_refuses_oversized_workspace_without_launching():
    """A call whose workspace exceeds the scratch is refused (BZ_ERR_SCRATCH)
    and writes nothing."""
    lib = L.lib()
    M, N, K = 32, 20480, 2560
    w, sc, _ = _int4(N, K, 8)
    x = _x(M, K, 9)
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    d = _desc(x, w, G.W_INT4_ZP, N, sc0=sc, out=out, path=4, slices=4)
    assert lib.bz_gemv_workspace(ctypes.byref(d)) > L.GEMV_SCRATCH_BYTES
    assert lib.bz_gemv_noalloc(ctypes.byref(d), L.stream_of(x)) == L.ERR_SCRATCH
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


def _capture_noalloc(calls):
    """Record bz_gemv_noalloc calls [(desc, x)] into one graph on a side stream."""
    lib = L.lib()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st), torch.cuda.graph(g, stream=st):
        for d, _ in calls:
            L.check(lib.bz_gemv_noalloc(ctypes.byref(d), st.cuda_stream), "bz_gemv_noalloc")
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    return g


def test_noalloc_under_graph_capture():
    """Tile-path calls (down K10240 N2560 at M = 16, then M = 6, split-K
    partials in the scratch) recorded into a HIP graph and replayed three
    times, with eager bz_gemv_noalloc and torch work between the replays:
    every replay gives bz_gemv's result bit for bit."""
    N, K = 2560, 10240
    w, sc, _ = _int4(N, K, 11)
    calls, refs, outs = [], [], []
    for m in (16, 6):
        x = _x(m, K, 40 + m)
        ref, _, need = _both(x, w, G.W_INT4_ZP, N, sc0=sc)
        assert need > 0
        out = torch.zeros(m, N, device="cuda", dtype=torch.bfloat16)
        calls.append((_desc(x, w, G.W_INT4_ZP, N, sc0=sc, out=out), x))
        refs.append(ref)
        outs.append(out)
    g = _capture_noalloc(calls)
    lib = L.lib()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), rep
        # eager use of the same scratch between replays (a shorter call)
        x = _x(5, K, 70 + rep)
        ref, got, _ = _both(x, w, G.W_INT4_ZP, N, sc0=sc)
        assert torch.equal(got, ref), rep
        torch.randn(1 << 20, device="cuda").sum().item()
    del g, lib


_FIRST_CALL_CHILD = r"""
import ctypes, sys
sys.path[:0] = [{root!r}, {pkg!r}]
import torch
from breeze_amd import _lib as L
from breeze_amd import gemv as G
torch.manual_seed(0)
N, K, M = 2560, 10240, 16
w = torch.randn(N, K, device="cuda") * 0.02
packed, sz, _ = G.quantize_int4_device(w, 128, True, G.W_INT4_ZP)
x = torch.randn(M, K, device="cuda").to(torch.bfloat16)
torch.cuda.synchronize()

def desc(out):
    d = L.GemvDesc()
    d.abi_version = L.ABI_VERSION
    d.M, d.N, d.K, d.group, d.wfmt = M, N, K, 128, G.W_INT4_ZP
    d.out_dtype = d.residual_dtype = L.DT_BF16
    d.eps = 1e-6
    d.x, d.ldx, d.w, d.sc0 = x.data_ptr(), x.stride(0), packed.data_ptr(), sz.data_ptr()
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    return d

lib = L.lib()
got = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
st = torch.cuda.Stream()
st.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
d = desc(got)
assert lib.bz_gemv_workspace(ctypes.byref(d)) > 0
with torch.cuda.stream(st), torch.cuda.graph(g, stream=st):
    # the process's first bz_gemv_noalloc call on this device, under capture
    rc = lib.bz_gemv_noalloc(ctypes.byref(d), st.cuda_stream)
torch.cuda.current_stream().wait_stream(st)
assert rc == 0, rc
ref = torch.empty_like(got)
dr = desc(ref)
ws = torch.zeros(lib.bz_gemv_workspace(ctypes.byref(dr)) // 4 + 4, dtype=torch.int32, device="cuda")
dr.workspace, dr.workspace_bytes = ws.data_ptr(), ws.numel() * 4
assert lib.bz_gemv(ctypes.byref(dr), L.stream_of(x)) == 0
for rep in range(3):
    got.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(got, ref), rep
print("FIRST_CALL_UNDER_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_under_capture_in_fresh_process():
    """In a fresh child process, the first bz_gemv_noalloc call (which looks
    up the device's scratch address and records its counter clear) is made
    under graph capture; the replays equal bz_gemv's result bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    code = _FIRST_CALL_CHILD.format(root=str(root), pkg=str(root / "breeze-tts-2_amd"))
    print("child: first bz_gemv_noalloc call under capture, K10240 N2560 M16", flush=True)
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    assert "FIRST_CALL_UNDER_CAPTURE_OK" in res.stdout
