"""The C ABI of libbzgemv.so without a GPU: the library loads, exports every
function the headers under include/ declare, the ctypes descriptor matches the C
struct byte for byte, and argument validation answers with the documented
status codes before anything touches a device."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bz_gemv.h"
HEADERS = tuple(sorted((ROOT / "include").glob("*.h")))


@pytest.fixture(scope="module")
def L():
    from breeze_amd import _lib

    if not _lib.LIB_PATH.exists():
        from breeze_amd import build

        build.build()
    return _lib


def declared_functions() -> list[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(bz_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_binding_exports(L):
    assert declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol(L):
    lib = L.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True, text=True).stdout
        syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
        for name in declared_functions():
            assert name in syms, name


def test_abi_version_matches_header(L):
    v = int(re.search(r"#define\s+BZ_ABI_VERSION\s+(\d+)", HEADER.read_text()).group(1))
    assert L.lib().bz_abi_version() == v == L.ABI_VERSION


def test_enum_values_match_header(L):
    pairs = re.findall(r"\b(BZ_[A-Z0-9_]+)\s*=\s*(\d+)", HEADER.read_text())
    assert len(pairs) >= 16
    for name, val in pairs:
        assert getattr(L, name[3:]) == int(val), name


def test_strerror(L):
    lib = L.lib()
    msgs = [lib.bz_strerror(i).decode() for i in range(8)]
    assert msgs[0] == "ok" and len(set(msgs)) == 8
    assert lib.bz_strerror(99).decode() == "unknown status"


def test_descriptor_layout_matches_c(L, tmp_path):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    fields = [f for f, _ in L.GemvDesc._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {",
           '  printf("size %zu\\n", sizeof(bz_gemv_desc));']
    src += [f'  printf("{f} %zu\\n", offsetof(bz_gemv_desc, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", str(c), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(L.GemvDesc)
    for f in fields:
        assert int(got[f]) == getattr(L.GemvDesc, f).offset, f


def _desc(L, **kw):
    d = L.GemvDesc()
    d.abi_version = L.ABI_VERSION
    d.M, d.N, d.K, d.group = 1, 64, 256, 128
    d.wfmt, d.epilogue, d.out_dtype = L.W_INT4_ZP, L.EPI_NONE, L.DT_BF16
    d.eps = 1e-6
    fake = 1 << 20  # never dereferenced: every case below fails validation
    d.x, d.ldx, d.w, d.sc0, d.out, d.ldo = fake, 256, fake, fake, fake, 64
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize(
    "kw,status",
    [
        ({"abi_version": 99}, "ERR_ABI"),
        ({"M": 0}, "ERR_INVALID_ARG"),
        ({"wfmt": 8}, "ERR_INVALID_ARG"),
        ({"wfmt": 4, "epilogue": 1}, "ERR_UNSUPPORTED"),       # plain tiled + SiLU-gate
        ({"wfmt": 5}, "ERR_UNSUPPORTED"),                      # paired tiled needs SiLU-gate
        ({"wfmt": 7}, "ERR_UNSUPPORTED"),
        ({"wfmt": 4, "N": 72}, "ERR_SHAPE"),                   # 16-row blocks
        ({"wfmt": 4, "K": 192, "ldx": 192}, "ERR_SHAPE"),      # int4 unit = 128 k
        ({"wfmt": 4, "group": 64}, "ERR_SHAPE"),               # tiled int4 is group 128
        ({"wfmt": 6, "K": 160, "ldx": 160}, "ERR_SHAPE"),      # fp8 unit = 64 k
        ({"wfmt": 4, "cfg_path": 2}, "ERR_UNSUPPORTED"),       # tiled formats run paths 4, 5 and 6 only
        ({"wfmt": 5, "epilogue": 1, "cfg_path": 4}, "ERR_UNSUPPORTED"),  # paired: streaming path only
        ({"wfmt": 4, "cfg_path": 4, "n_out2": 8, "out2": 1 << 20, "ldo2": 8}, "ERR_UNSUPPORTED"),  # no second store
        ({"cfg_path": 5}, "ERR_UNSUPPORTED"),                  # path 5 reads tiled formats only
        ({"cfg_path": 6}, "ERR_UNSUPPORTED"),                  # path 6 reads tiled formats only
        ({"cfg_path": 7}, "ERR_INVALID_ARG"),
        ({"wfmt": 4, "cfg_path": 6, "gamma": 1 << 20}, "ERR_UNSUPPORTED"),          # panel: no RMSNorm
        ({"wfmt": 5, "epilogue": 1, "cfg_path": 6}, "ERR_UNSUPPORTED"),            # ... no paired weights
        ({"wfmt": 4, "cfg_path": 6, "n_out2": 8, "out2": 1 << 20, "ldo2": 8}, "ERR_UNSUPPORTED"),  # ... no 2nd store
        ({"wfmt": 4, "cfg_path": 6, "cfg_tiles": 6}, "ERR_INVALID_ARG"),           # ... 1-5 blocks
        ({"wfmt": 4, "cfg_path": 6, "cfg_waves": 17}, "ERR_INVALID_ARG"),          # ... <= 16 waves
        ({"wfmt": 4, "cfg_path": 6, "cfg_tiles": 2, "cfg_waves": 9}, "ERR_INVALID_ARG"),  # ... 8 with blocks
        ({"wfmt": 6, "K": 704, "ldx": 704, "cfg_path": 6, "cfg_waves": 1}, "ERR_UNSUPPORTED"),  # 11 units a wave
        ({"reserved0": 1}, "ERR_INVALID_ARG"),
        ({"n_out2": 8, "out2": 1 << 20, "ldo2": 8}, "ERR_UNSUPPORTED"),            # second store: tiled only
        ({"wfmt": 4, "n_out2": 8, "ldo2": 8}, "ERR_INVALID_ARG"),                # ... needs out2
        ({"wfmt": 4, "n_out2": 65, "out2": 1 << 20, "ldo2": 65}, "ERR_INVALID_ARG"),  # ... at most N_out
        ({"wfmt": 4, "n_out2": 8, "out2": 1 << 20, "ldo2": 4}, "ERR_INVALID_ARG"),   # ... ldo2 >= n_out2
        ({"wfmt": 4, "n_out2": -1}, "ERR_INVALID_ARG"),
        ({"wfmt": 4, "n_out2": 8, "out2": (1 << 20) + 1, "ldo2": 8}, "ERR_ALIGNMENT"),
        ({"wfmt": 4, "w": (1 << 20) + 8}, "ERR_ALIGNMENT"),
        ({"epilogue": 5}, "ERR_INVALID_ARG"),
        ({"out_dtype": 3}, "ERR_INVALID_ARG"),
        ({"x": None}, "ERR_INVALID_ARG"),
        ({"sc0": None}, "ERR_INVALID_ARG"),
        ({"wfmt": 1}, "ERR_INVALID_ARG"),                      # INT4_MIN needs sc1
        ({"epilogue": 2}, "ERR_INVALID_ARG"),                  # RESIDUAL needs residual
        ({"K": 200}, "ERR_SHAPE"),                             # K % group
        ({"group": 96}, "ERR_SHAPE"),                          # not a power of two
        ({"group": 16, "K": 256}, "ERR_SHAPE"),                # below 32
        ({"epilogue": 1, "N": 63}, "ERR_SHAPE"),               # SiLU-gate needs even N
        ({"wfmt": 2, "K": 264}, "ERR_SHAPE"),                  # fp8 K % 16
        ({"wfmt": 3, "K": 260}, "ERR_SHAPE"),                  # bf16 K % 8
        ({"ldx": 100}, "ERR_INVALID_ARG"),                     # ldx < K
        ({"x": (1 << 20) + 2}, "ERR_ALIGNMENT"),
        ({"w": (1 << 20) + 8}, "ERR_ALIGNMENT"),
        ({"ldx": 260}, "ERR_ALIGNMENT"),                       # rows not 16-byte aligned
        ({"cfg_path": 4}, "ERR_INVALID_ARG"),
        ({"cfg_path": 3, "wfmt": 2}, "ERR_UNSUPPORTED"),               # int8 path is int4-only
        ({"cfg_path": 3, "group": 64}, "ERR_UNSUPPORTED"),             # and needs group >= 128
        ({"cfg_path": 3, "cfg_depth": 16}, "ERR_INVALID_ARG"),         # int8 path: depth <= 8
        ({"cfg_tiles": -1}, "ERR_INVALID_ARG"),
        ({"cfg_depth": 3}, "ERR_INVALID_ARG"),
        ({"cfg_depth": 16, "epilogue": 1}, "ERR_INVALID_ARG"),  # 2 x 16 loads in flight
        ({"cfg_waves": 9}, "ERR_INVALID_ARG"),
        ({"group": 64, "cfg_path": 2}, "ERR_UNSUPPORTED"),      # MFMA path needs group >= 128
    ],
)
def test_gemv_validation(L, kw, status):
    d = _desc(L, **kw)
    assert L.lib().bz_gemv(ctypes.byref(d), None) == getattr(L, status)


def test_tiled_bytes(L):
    """Row blocks x chunk: int4 NU x (1024 + 64) bytes, fp8 NU x 1024 + 64,
    each rounded up to 128; 0 for untileable shapes."""
    tb = L.lib().bz_tiled_bytes
    assert tb(L.W_INT4_TILED, 20480, 2560) == 1280 * 20 * 1088
    assert tb(L.W_INT4_TILED_PAIRED, 20480, 2560) == 1280 * 20 * 1088
    assert tb(L.W_INT4_TILED, 16, 128) == 1152           # 1088 -> 1152
    assert tb(L.W_FP8_TILED, 2560, 10240) == 160 * (160 * 1024 + 128)
    assert tb(L.W_FP8_TILED_PAIRED, 32, 64) == 2 * 1152
    assert tb(L.W_INT4_TILED, 24, 128) == 0              # rows % 16
    assert tb(L.W_INT4_TILED, 16, 64) == 0               # K % 128
    assert tb(L.W_FP8_TILED, 16, 96) == 0                # K % 64
    assert tb(L.W_INT4_ZP, 16, 128) == 0                 # not a tiled format


@pytest.mark.parametrize(
    "args,status",
    [
        ((0, 0, 1 << 20, 16, 256, 128, 4, 1 << 20, 16, 0), "ERR_INVALID_ARG"),   # null source
        ((0, 1 << 20, 1 << 20, 16, 256, 128, 0, 1 << 20, 16, 0), "ERR_INVALID_ARG"),  # dst not tiled
        ((2, 1 << 20, 1 << 20, 16, 256, 128, 4, 1 << 20, 16, 0), "ERR_INVALID_ARG"),  # fp8 source, int4 dst
        ((0, 1 << 20, None, 16, 256, 128, 4, 1 << 20, 16, 0), "ERR_INVALID_ARG"),     # row-major needs scales
        ((0, 1 << 20, 1 << 20, 16, 256, 128, 4, 1 << 20, 16, 8), "ERR_INVALID_ARG"),  # rows past N
        ((0, 1 << 20, 1 << 20, 16, 256, 64, 4, 1 << 20, 16, 0), "ERR_SHAPE"),         # group 64
        ((0, 1 << 20, 1 << 20, 24, 256, 128, 4, 1 << 20, 24, 0), "ERR_SHAPE"),        # N % 16
        ((4, 1 << 20, None, 8, 256, 128, 5, 1 << 20, 16, 0), "ERR_SHAPE"),            # tiled source rows % 16
        ((0, (1 << 20) + 4, 1 << 20, 16, 256, 128, 4, 1 << 20, 16, 0), "ERR_ALIGNMENT"),
        ((0, 1 << 20, (1 << 20) + 2, 16, 256, 128, 4, 1 << 20, 16, 0), "ERR_ALIGNMENT"),
    ],
)
def test_pack_tiled_validation(L, args, status):
    assert L.lib().bz_pack_tiled(*args, None) == getattr(L, status)


def test_gemv_null_descriptor(L):
    assert L.lib().bz_gemv(None, None) == L.ERR_INVALID_ARG


def test_workspace_sizes(L):
    """0 below 5 rows, with an RMSNorm or a SiLU gate, or for an invalid
    descriptor; otherwise the counters (16 KB) plus nsl x N x MP fp32
    partials of the several-row tile path (MP = M rounded up to 4)."""
    ws = lambda **kw: L.lib().bz_gemv_workspace(ctypes.byref(_desc(L, **kw)))  # noqa: E731
    assert ws() == 0
    assert ws(M=4) == 0
    # N = 64: one column block, so the rule asks for the most slices: K / 128 = 2
    assert ws(M=8) == 16384 + 2 * 8 * 64 * 4
    assert ws(M=32, K=1024, ldx=1024) == 16384 + 8 * 32 * 64 * 4
    assert ws(M=40, K=1024, ldx=1024) == 16384 + 8 * 32 * 64 * 4  # 32 rows per launch
    assert ws(M=8, gamma=1 << 20) == 0
    assert ws(M=8, N=128, epilogue=1) == 0
    assert ws(M=8, abi_version=99) == 0
    assert ws(M=2, cfg_path=4, cfg_slices=1) == 0              # one slice: no partials
    assert ws(M=2, cfg_path=4, cfg_slices=2) == 16384 + 2 * 4 * 64 * 4   # rows padded to 4
    assert ws(M=6, cfg_path=4, cfg_slices=2) == 16384 + 2 * 8 * 64 * 4


@pytest.mark.parametrize(
    "kw,status",
    [
        ({"cfg_path": 6}, "ERR_UNSUPPORTED"),                  # path 6 reads tiled formats only
        ({"cfg_path": 7}, "ERR_INVALID_ARG"),
        ({"wfmt": 4, "cfg_path": 6, "gamma": 1 << 20}, "ERR_UNSUPPORTED"),          # panel: no RMSNorm
        ({"wfmt": 5, "epilogue": 1, "cfg_path": 6}, "ERR_UNSUPPORTED"),            # ... no paired weights
        ({"wfmt": 4, "cfg_path": 6, "n_out2": 8, "out2": 1 << 20, "ldo2": 8}, "ERR_UNSUPPORTED"),  # ... no 2nd store
        ({"wfmt": 4, "cfg_path": 6, "cfg_tiles": 6}, "ERR_INVALID_ARG"),           # ... 1-5 blocks
        ({"wfmt": 4, "cfg_path": 6, "cfg_waves": 17}, "ERR_INVALID_ARG"),          # ... <= 16 waves
        ({"wfmt": 4, "cfg_path": 6, "cfg_tiles": 2, "cfg_waves": 9}, "ERR_INVALID_ARG"),  # ... 8 with blocks
        ({"wfmt": 6, "K": 704, "ldx": 704, "cfg_path": 6, "cfg_waves": 1}, "ERR_UNSUPPORTED"),  # 11 units a wave
        ({"reserved0": 1}, "ERR_INVALID_ARG"),
        ({"n_out2": 8, "out2": 1 << 20, "ldo2": 8}, "ERR_UNSUPPORTED"),            # second store: tiled only
        ({"wfmt": 4, "n_out2": 8, "ldo2": 8}, "ERR_INVALID_ARG"),                # ... needs out2
        ({"wfmt": 4, "n_out2": 65, "out2": 1 << 20, "ldo2": 65}, "ERR_INVALID_ARG"),  # ... at most N_out
        ({"wfmt": 4, "n_out2": 8, "out2": 1 << 20, "ldo2": 4}, "ERR_INVALID_ARG"),   # ... ldo2 >= n_out2
        ({"wfmt": 4, "n_out2": -1}, "ERR_INVALID_ARG"),
        ({"wfmt": 4, "n_out2": 8, "out2": (1 << 20) + 1, "ldo2": 8}, "ERR_ALIGNMENT"),
        ({"cfg_path": 4, "M": 8}, "ERR_INVALID_ARG"),                       # split-K needs the workspace
        ({"cfg_path": 4, "M": 8, "workspace": 1 << 20, "workspace_bytes": 100}, "ERR_INVALID_ARG"),
        ({"cfg_path": 4, "M": 8, "cfg_tiles": 3}, "ERR_INVALID_ARG"),
        ({"cfg_path": 4, "M": 8, "cfg_waves": 6}, "ERR_INVALID_ARG"),
        ({"cfg_slices": -1}, "ERR_INVALID_ARG"),
        ({"cfg_path": 4, "M": 8, "cfg_depth": 16}, "ERR_INVALID_ARG"),
        ({"cfg_path": 4, "M": 8, "gamma": 1 << 20}, "ERR_UNSUPPORTED"),     # no RMSNorm prologue
        ({"cfg_path": 4, "M": 8, "N": 128, "epilogue": 1}, "ERR_UNSUPPORTED"),  # no SiLU gate
        ({"cfg_path": 4, "M": 8, "group": 64}, "ERR_UNSUPPORTED"),          # int4 group >= 128
        ({"cfg_path": 4, "M": 8, "wfmt": 2, "K": 272, "ldx": 272}, "ERR_UNSUPPORTED"),  # fp8 K % 64
    ],
)
def test_tile_path_validation(L, kw, status):
    d = _desc(L, **kw)
    assert L.lib().bz_gemv(ctypes.byref(d), None) == getattr(L, status)


def test_aux_validation(L):
    lib = L.lib()
    f = 1 << 20
    assert lib.bz_rmsnorm(None, 8, f, 1e-6, f, 8, 1, 8, None) == L.ERR_INVALID_ARG
    assert lib.bz_rmsnorm(f, 4, f, 1e-6, f, 8, 1, 8, None) == L.ERR_INVALID_ARG
    assert lib.bz_silu_mul(f, 8, f, 8, f, 8, 0, 8, None) == L.ERR_INVALID_ARG
    assert lib.bz_quantize_int4(f, 1, 8, 256, 96, 0, 0, f, f, None, None) == L.ERR_SHAPE
    assert lib.bz_quantize_int4(f, 1, 8, 256, 128, 0, 1, f, f, None, None) == L.ERR_INVALID_ARG
    assert lib.bz_quantize_int4(f, 5, 8, 256, 128, 0, 0, f, f, None, None) == L.ERR_INVALID_ARG
    assert lib.bz_quantize_fp8(f, 5, 8, 256, 1e-12, f, f, None) == L.ERR_INVALID_ARG
    assert lib.bz_dequant(0, f, f, None, 8, 200, 128, f, None) == L.ERR_SHAPE
    assert lib.bz_dequant(0, f + 4, f, None, 8, 256, 128, f, None) == L.ERR_ALIGNMENT
    assert lib.bz_dequant(9, f, f, None, 8, 256, 128, f, None) == L.ERR_INVALID_ARG


def _rope_args(L, **kw):
    f = 1 << 20
    a = dict(qkv=f, ld_qkv=24 * 64, B=1, HQ=16, HKV=4, D=64, qn=f, kn=f, eps=1e-6, cos=f, sin=f, cs_dtype=L.DT_BF16,
             ld_cs=64, pos=f, q_out=f, kc=f, vc=f, S=32, cache_dtype=L.DT_BF16, seq_len=None, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize(
    "kw,status",
    [
        ({"qkv": None}, "ERR_INVALID_ARG"),
        ({"pos": None}, "ERR_INVALID_ARG"),
        ({"kn": None}, "ERR_INVALID_ARG"),        # q and k norm weights come together
        ({"HKV": 0}, "ERR_INVALID_ARG"),
        ({"cs_dtype": 2}, "ERR_INVALID_ARG"),
        ({"cache_dtype": 2}, "ERR_INVALID_ARG"),
        ({"D": 63}, "ERR_SHAPE"),
        ({"D": 2048, "ld_qkv": 24 * 2048}, "ERR_SHAPE"),
        ({"ld_qkv": 24 * 64 - 1}, "ERR_SHAPE"),
        ({"ld_cs": -1}, "ERR_SHAPE"),
    ],
)
def test_rope_cache_validation(L, kw, status):
    assert L.lib().bz_qkv_rope_cache(*_rope_args(L, **kw)) == getattr(L, status)


def _attn_args(L, **kw):
    f = 1 << 20
    a = dict(q=f, kc=f, vc=f, cache_dtype=L.DT_BF16, B=2, HQ=16, HKV=4, D=256, S=512, mask=f, mask_dtype=L.DT_BF16,
             ld_mask=512, pos=f, scale=0.0625, split=4, ws=f, out=f, ld_out=4096, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize(
    "kw,status",
    [
        ({"q": None}, "ERR_INVALID_ARG"),
        ({"mask": None}, "ERR_INVALID_ARG"),
        ({"HQ": 15}, "ERR_INVALID_ARG"),                 # HQ % HKV
        ({"cache_dtype": 3}, "ERR_INVALID_ARG"),
        ({"mask_dtype": 3}, "ERR_INVALID_ARG"),
        ({"ld_mask": -1}, "ERR_SHAPE"),
        ({"split": 0}, "ERR_INVALID_ARG"),
        ({"split": 65}, "ERR_INVALID_ARG"),
        ({"ws": None}, "ERR_INVALID_ARG"),               # split > 1 needs the workspace
        ({"ws": (1 << 20) + 2}, "ERR_ALIGNMENT"),
        ({"ld_mask": 100}, "ERR_SHAPE"),
        ({"ld_out": 4095}, "ERR_SHAPE"),
        ({"D": 96, "ld_out": 16 * 96}, "ERR_UNSUPPORTED"),
        ({"HQ": 32, "HKV": 1, "ld_out": 32 * 256}, "ERR_UNSUPPORTED"),   # G > 16
        ({"D": 512, "HKV": 2, "ld_out": 16 * 512}, "ERR_UNSUPPORTED"),   # G > 4 at D = 512
        ({"q": (1 << 20) + 4}, "ERR_ALIGNMENT"),
        ({"kc": (1 << 20) + 8}, "ERR_ALIGNMENT"),
    ],
)
def test_attn_validation(L, kw, status):
    assert L.lib().bz_attn_decode(*_attn_args(L, **kw)) == getattr(L, status)


def _step_args(L, **kw):
    f = 1 << 20
    a = dict(qkv=f, ld_qkv=24 * 256, B=2, HQ=16, HKV=4, D=256, qn=f, kn=f, eps=1e-6, cos=f, sin=f,
             cs_dtype=L.DT_BF16, ld_cs=256, pos=f, kc=f, vc=f, S=512, cache_dtype=L.DT_BF16, seq_len=None, mask=f,
             mask_dtype=L.DT_BF16, ld_mask=512, scale=0.0625, split=4, ws=f, out=f, ld_out=4096, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize(
    "kw,status",
    [
        ({"qkv": None}, "ERR_INVALID_ARG"),
        ({"cos": None}, "ERR_INVALID_ARG"),
        ({"qn": None}, "ERR_INVALID_ARG"),             # q and k norm weights come together
        ({"cs_dtype": 2}, "ERR_INVALID_ARG"),
        ({"ld_qkv": 24 * 256 - 8}, "ERR_SHAPE"),
        ({"ld_cs": -1}, "ERR_SHAPE"),
        ({"HQ": 15}, "ERR_INVALID_ARG"),
        ({"ws": None}, "ERR_INVALID_ARG"),
        ({"D": 96, "ld_qkv": 24 * 96, "ld_out": 16 * 96}, "ERR_UNSUPPORTED"),
        ({"kc": (1 << 20) + 8}, "ERR_ALIGNMENT"),
    ],
)
def test_attn_step_validation(L, kw, status):
    assert L.lib().bz_attn_step(*_step_args(L, **kw)) == getattr(L, status)


def test_attn_header_constants(L):
    text = (ROOT / "include" / "bz_attn.h").read_text()
    assert int(re.search(r"#define\s+BZ_MASK_BOOL\s+(\d+)", text).group(1)) == L.MASK_BOOL
    assert int(re.search(r"#define\s+BZ_ATTN_MAX_SPLIT\s+(\d+)", text).group(1)) == 64


def test_attn_workspace_and_split(L):
    lib = L.lib()
    assert lib.bz_attn_workspace(2, 16, 4, 256, 1) == 0
    assert lib.bz_attn_workspace(2, 16, 4, 256, 8) == 2 * 16 * 8 * 260 * 4 + 2 * 4 * 4
    assert [lib.bz_attn_default_split(s) for s in (1, 128, 129, 1024, 2048, 8192)] == [1, 1, 2, 8, 16, 32]


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from breeze_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()


def test_head_f32_validation(L):
    lib = L.lib()
    f = 1 << 20
    args = dict(x=f, ldx=1024, M=2, K=1024, w=f, N=2051, stride=2051 * 1024, nmat=15, index=None, off=0, out=f,
                ldo=2051, stream=None)

    def call(**kw):
        a = dict(args)
        a.update(kw)
        return lib.bz_head_f32(*a.values())

    assert call(x=None) == L.ERR_INVALID_ARG
    assert call(M=0) == L.ERR_INVALID_ARG
    assert call(nmat=0) == L.ERR_INVALID_ARG
    assert call(K=1022, ldx=1024) == L.ERR_SHAPE          # K % 4
    assert call(K=8192, ldx=8192) == L.ERR_SHAPE          # beyond the LDS staging of x
    assert call(stride=100) == L.ERR_SHAPE                # matrices overlap
    assert call(ldo=2000) == L.ERR_SHAPE
    assert call(w=f + 4) == L.ERR_ALIGNMENT


def _sample_args(L, **kw):
    fake = 1 << 20  # never dereferenced: every case below fails validation
    a = dict(logits=fake, ld=2051, B=2, V=2051, codec=2048, max_k=1024, guidance=fake, temperature=fake,
             top_k=fake, top_p=fake, do_sample=fake, seed=fake, counters=fake, tokens=fake, cfg_out=None,
             probs_out=None, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize(
    "kw",
    [
        {"B": 3},                      # CFG rows come in pairs
        {"B": 0},
        {"V": 4097, "ld": 4097},       # wider than the sort
        {"ld": 2000},                  # row stride below V
        {"codec": 0},
        {"codec": 2052},
        {"max_k": 0},
        {"max_k": 1025},               # one rank per thread
        {"V": 64, "ld": 64, "codec": 64, "max_k": 65},  # wider than the vocabulary
        {"guidance": None},            # CFG needs it
        {"seed": None},
        {"counters": None},
        {"tokens": None},
        {"logits": None},
    ],
)
def test_sample_validation(L, kw):
    assert L.lib().bz_sample_cfg(*_sample_args(L, **kw)) == L.ERR_INVALID_ARG


def test_gemv_noalloc_refuses_before_touching_the_gpu(L):
    """bz_gemv_noalloc checks the descriptor version and its workspace need
    against BZ_GEMV_SCRATCH_BYTES before any HIP call: both refusals work
    without a GPU."""
    lib = L.lib()
    assert lib.bz_gemv_noalloc(None, None) == L.ERR_INVALID_ARG
    assert lib.bz_gemv_noalloc(ctypes.byref(_desc(L, abi_version=99)), None) == L.ERR_ABI
    # forced split-K tile path whose partials (4 slices x 32 x 20480 fp32) exceed 8 MiB
    big = _desc(L, M=32, N=20480, K=2560, ldx=2560, ldo=20480, cfg_path=4, cfg_slices=4)
    assert lib.bz_gemv_workspace(ctypes.byref(big)) > L.GEMV_SCRATCH_BYTES
    assert lib.bz_gemv_noalloc(ctypes.byref(big), None) == L.ERR_SCRATCH
    assert "BZ_GEMV_SCRATCH_BYTES" in lib.bz_strerror(L.ERR_SCRATCH).decode()
    header = HEADER.read_text()
    assert re.search(r"#define BZ_GEMV_SCRATCH_BYTES \(\(size_t\)8 << 20\)", header)
    assert L.GEMV_SCRATCH_BYTES == 8 << 20


def test_stream_read_validation(L):
    """The read-floor kernel's argument checks (no launch happens)."""
    lib = L.lib()
    fake = 1 << 20
    assert lib.bz_stream_read(fake, 4096, 1024, 0, None, None) == L.ERR_INVALID_ARG     # no sink
    assert lib.bz_stream_read(None, 4096, 1024, 0, fake, None) == L.ERR_INVALID_ARG     # no buffer
    assert lib.bz_stream_read(fake, 4096, 0, 0, fake, None) == L.ERR_INVALID_ARG        # no chunk
    assert lib.bz_stream_read(fake, 4096, 1000, 0, fake, None) == L.ERR_SHAPE           # bytes % chunk
    assert lib.bz_stream_read(fake, 4104, 1368, 0, fake, None) == L.ERR_SHAPE           # chunk % 16
    assert lib.bz_stream_read(fake + 8, 4096, 1024, 0, fake, None) == L.ERR_ALIGNMENT


def test_shared_read_validation(L):
    """The whole-K read floor's argument checks (no launch happens)."""
    lib = L.lib()
    fake = 1 << 20
    assert lib.bz_shared_read(fake, 4096, fake, 1024, 4, 0, None, None) == L.ERR_INVALID_ARG   # no sink
    assert lib.bz_shared_read(None, 4096, fake, 1024, 4, 0, fake, None) == L.ERR_INVALID_ARG   # no x
    assert lib.bz_shared_read(fake, 4096, None, 1024, 4, 0, fake, None) == L.ERR_INVALID_ARG   # chunk, no w
    assert lib.bz_shared_read(fake, 4096, fake, 1024, 0, 0, fake, None) == L.ERR_INVALID_ARG   # no workgroups
    assert lib.bz_shared_read(fake, 0, fake, 1024, 4, 0, fake, None) == L.ERR_SHAPE            # no x bytes
    assert lib.bz_shared_read(fake, 4100, fake, 1024, 4, 0, fake, None) == L.ERR_SHAPE         # x % 16
    assert lib.bz_shared_read(fake, 4096, fake, 1000, 4, 0, fake, None) == L.ERR_SHAPE         # chunk % 16
    assert lib.bz_shared_read(fake, (64 << 20) + 16, fake, 0, 4, 0, fake, None) == L.ERR_SHAPE
    assert lib.bz_shared_read(fake, 4096, fake, (16 << 20) + 16, 4, 0, fake, None) == L.ERR_SHAPE
    assert lib.bz_shared_read(fake + 8, 4096, fake, 1024, 4, 0, fake, None) == L.ERR_ALIGNMENT
    assert lib.bz_shared_read(fake, 4096, fake + 8, 1024, 4, 0, fake, None) == L.ERR_ALIGNMENT
    assert lib.bz_shared_read(fake, 4096, fake, 1024, 65537, 0, fake, None) == L.ERR_UNSUPPORTED
