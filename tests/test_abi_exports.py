"""CPU-side checks of the drop-in boundary: the built libg1env.so loads and exports every symbol
include/g1env.h declares (no compute calls: there is no GPU here), and the header's reference
surface matches the reference's extern "C" list (src/g1_env.cu:361-476)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "g1env.h")
LIB = os.path.join(ROOT, "g1.cu_amd", "build", "libg1env.so")

REFERENCE_SURFACE = ["g1_env_create", "g1_env_reset", "g1_env_step", "g1_rollout", "g1_env_qpos", "g1_env_qpos_all",
                     "g1_env_bench_phys", "g1_occupancy_report", "g1_env_obs_dim", "g1_env_act_dim",
                     "g1_env_destroy"]


def declared():
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:void\*|void|int|long)\s+(g1_\w+)\s*\(", text, re.M)


def test_header_declares_reference_surface():
    names = declared()
    for n in REFERENCE_SURFACE:
        assert n in names, n


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.skip("libg1env.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    # dimension queries touch no device
    lib.g1_env_obs_dim.restype = ctypes.c_int
    lib.g1_env_act_dim.restype = ctypes.c_int
    assert lib.g1_env_obs_dim() == 100 and lib.g1_env_act_dim() == 29


def test_ppo_binding_argtypes_match_reference_driver():
    """The fused entry point is bound exactly as the reference driver binds it
    (scripts/ppo_fused.py:27-28): (c_void_p, c_int) + 10 x c_void_p, restype None."""
    text = open(os.path.join(ROOT, "g1.cu_amd", "scripts", "ppo.py")).read()
    assert "_lib.g1_rollout.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 10" in text
    assert "_lib.g1_env_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_ulong]" in text
