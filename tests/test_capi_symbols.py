"""The C ABI: every entry point declared in include/tu_hip.h is exported by
libtu_hip.so and described identically (argument count, return type) in the
ctypes binding.  Nothing here launches GPU work."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from comfyui_turing_utils_kernel import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tu_hip.h")


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"(const char \*|int32_t|int64_t)\s*(tu_\w+)\(([^)]*)\);", text):
        args = args.strip()
        n = 0 if args in ("", "void") else len(args.split(","))
        out[name] = (ret.strip(), n)
    return out


def test_header_parses():
    decls = _declarations()
    assert len(decls) >= 11
    assert "tu_sage_attn_fwd" in decls and "tu_int8_gemm_bf16" in decls


def test_binding_matches_header():
    decls = _declarations()
    assert set(decls) == set(_lib.SIGNATURES)
    for name, (ret, nargs) in decls.items():
        restype, argtypes = _lib.SIGNATURES[name]
        assert len(argtypes) == nargs, name
        expected = {"int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64}.get(ret, ctypes.c_char_p)
        assert restype is expected, name


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is missing: {_lib.BUILD_HINT}")
    return _lib.load()


def test_library_exports_every_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    missing = set(_declarations()) - exported
    assert not missing, missing
    for name in _declarations():
        assert hasattr(lib, name)


def test_abi_version_and_error_channel(lib):
    assert lib.tu_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.tu_last_error(), bytes)


def test_argument_errors_are_reported_without_launching(lib):
    """Shape checks run on the host before any HIP call: a bad group size is
    rejected with a message, and no device is touched."""
    rc = lib.tu_convrot_quant_i8(None, None, None, 4, 100, 96, 0, None)
    assert rc != 0
    assert b"group" in lib.tu_last_error().lower()


def test_attention_key_split_plan(lib):
    """The split planner is host arithmetic: 256 workgroups a round, each
    costing its key tiles plus a fixed part.  Config 2 (1.5 rounds) splits in
    two, the bench shape (20 full rounds) and full grids do not, a grid of
    half a round splits, causal never does, and every range keeps >= 16 key
    tiles."""
    plan = lambda b, h, lq, lk, causal=0, cus=256: lib.tu_sage_attn_kv_splits(b, h, lq, lk, causal, cus)  # noqa: E731
    assert plan(1, 12, 8190, 8190) == 2
    assert plan(1, 40, 32760, 32760) == 1
    assert plan(1, 40, 8190, 8190) == 1
    assert plan(2, 12, 8190, 8190) == 1
    assert plan(1, 8, 4096, 4096) == 2
    assert plan(1, 12, 8190, 8190, causal=1) == 1
    assert plan(1, 1, 256, 64 * 20) == 1  # two ranges would hold 10 tiles each
    for b, h, lq, lk in [(1, 2, 100000, 100000), (1, 3, 300, 50000), (1, 1, 256, 64 * 32)]:
        n = plan(b, h, lq, lk)
        tiles = (lk + 63) // 64
        assert 1 <= n <= 8 and (n == 1 or (tiles + n - 1) // n >= 16)


def test_gemm_tile_policy_plan(lib):
    """The GEMM's tile policy is host arithmetic over rounds of one workgroup
    per CU: the four config-4 shapes (10-30 full rounds of 256 x 256 tiles)
    keep them; grids of a few partly empty rounds take 128 x 256 tiles (each
    round 0.635 of a 256 x 256 round, measured) or 256 x 192 tiles (0.85)
    when their rounds cost less: config 1 takes 256 x 192 (3 rounds of them
    against 3 of 256 x 256), the cross-attention's 512-row kv projection
    128-row tiles; bad arguments fall back to 256 x 256.  tu_int8_gemm_ex
    refuses an unknown policy or output type before any HIP call."""
    pol = lambda m, n, cus=256: lib.tu_int8_gemm_tile_policy(m, n, cus)  # noqa: E731
    for n in (15360, 5120, 13824):
        assert pol(32760, n) == 1
    assert pol(4096, 8960) == 3                  # config 1: 3 rounds x 0.85 against 3
    assert pol(2048, 8960) == 3                  # 2 x 0.85 against 2 (and 3 x 0.635)
    assert pol(512, 10240) == 2                  # 1 x 0.635 against 1 x 0.85 and 1
    assert pol(256 * 16, 256 * 16) == 1          # exactly one full round
    assert pol(0, 8960) == 1 and pol(4096, 8960, 0) == 1
    ceil = lambda a, b: -(-a // b)  # noqa: E731
    for m, n in ((4096, 8960), (8192, 8960), (2048, 3072), (32760, 15360), (300, 264), (4096, 5120), (512, 10240)):
        # the rule: the cheapest of the three by rounds x the tile's round cost
        c256 = ceil(ceil(m, 256) * ceil(n, 256), 256)
        c128 = ceil(ceil(m, 128) * ceil(n, 256), 256) * 0.635
        c192 = ceil(ceil(m, 256) * ceil(n, 192), 256) * 0.85
        want = 2 if (c128 < c256 and c128 <= c192) else 3 if c192 < c256 else 1
        assert pol(m, n) == want, (m, n)
    assert lib.tu_int8_gemm_ex(None, None, None, None, None, None, 0, 16, 16, 16, 4, None) != 0
    assert b"tile_policy" in lib.tu_last_error()
    assert lib.tu_int8_gemm_ex(None, None, None, None, None, None, 7, 16, 16, 16, 0, None) != 0


def test_attention_split_arguments_are_refused_on_the_host(lib):
    """tu_sage_attn_fwd_split checks its split count and workspace before any
    HIP call: more ranges than key tiles, more than 256, or a missing or
    short workspace are errors with a message."""
    def call(kv_splits, partial, nbytes, lk=4096):
        return lib.tu_sage_attn_fwd_split(
            None, None, 128, None, None, 128, None, 4096, None, 1, 8, 8, 4096, lk, 128,
            0, 0, 0, 0, 0, 0, 0, 0, 0, 0.088, kv_splits, partial, nbytes, None)
    assert call(65, 16, 1 << 30) != 0 and b"kv_splits" in lib.tu_last_error()     # 64 key tiles
    assert call(300, 16, 1 << 30, lk=1 << 20) != 0 and b"256" in lib.tu_last_error()
    assert call(0, 16, 1 << 30) != 0 and b"kv_splits" in lib.tu_last_error()
    assert call(2, None, 1 << 30) != 0 and b"workspace" in lib.tu_last_error()
    need = 2 * 1 * 8 * 4096 * (128 + 2) * 4
    assert call(2, 16, need - 4) != 0 and str(need).encode() in lib.tu_last_error()


def test_package_import_fails_loudly_without_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="libtu_hip|build"):
        _lib.load()
