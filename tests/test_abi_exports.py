"""The C-ABI library (no GPU needed): it loads, exports every function that
include/*.h declares, and the ctypes table in rapidllm_amd/hip.py agrees with the
header's parameter counts.  No compute call is made."""
import glob
import os
import re

import pytest

from rapidllm_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(rl_hip_\w+)\s*\(([^;{]*?)\)\s*;", re.M | re.S)


def declarations():
    out = {}
    for h in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))):
        text = re.sub(r"//[^\n]*", "", open(h).read())
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for name, params in DECL.findall(text):
            params = " ".join(params.split())
            out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


DECLS = declarations()


def test_header_declares_the_abi():
    assert len(DECLS) >= 60
    for must in ("rl_hip_gemm_fp8_frag", "rl_hip_gemm_kquant", "rl_hip_gdn_decode", "rl_hip_attn_decode_layer",
                 "rl_hip_argmax_rows", "rl_hip_accept_prefix", "rl_hip_engine_create", "rl_hip_engine_spec_verify"):
        assert must in DECLS


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(hip.LIB_PATH):
        pytest.skip("library not built (python -c 'import __graft_entry__ as g; g.build()')")
    return hip.lib()


def test_every_declared_symbol_is_exported(L):
    missing = [n for n in DECLS if not hasattr(L, n)]
    assert not missing, missing


def test_ctypes_table_matches_header(L):
    for name, nparams in DECLS.items():
        assert name in hip._SIGS, f"{name} has no ctypes signature"
        assert len(hip._SIGS[name][1]) == nparams, name
    extra = set(hip._SIGS) - set(DECLS)
    assert not extra, f"ctypes entries not in the header: {extra}"


def test_abi_version_and_status_without_gpu(L):
    assert L.rl_hip_abi_version() >= 1
    assert L.rl_hip_available() in (0, 1)
