"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/aic_hip.h declares, its host-side routines agree with the oracle, and argument
errors come back as codes (no GPU needed, no kernel launched)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import autonomousaicore_amd as aic
from autonomousaicore_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "aic_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aic_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = aic.load()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_version_and_device_count():
    lib = aic.load()
    assert b"gfx950" in lib.aic_hip_version()
    assert lib.aic_hip_device_count() >= 0


def test_argument_errors_are_codes():
    lib = aic.load()
    rc = lib.aic_hip_gemm(0, 1, -1, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None, 0, _lib.AIC_BF16,
                          _lib.AIC_BF16, None)
    assert rc == 1  # InvalidArgument
    assert b"negative" in lib.aic_hip_last_error()
    rc = lib.aic_hip_rope(None, 8, 1, 1, 1, 7, 0, None, None, 0, _lib.AIC_F32, None)
    assert rc == 1 and b"even" in lib.aic_hip_last_error()
    rc = lib.aic_hip_embed_bwd(None, (1 << 20) + 1, None, 10, 4, None, 0, _lib.AIC_F32, None)
    assert rc == 1 and b"tokens per call" in lib.aic_hip_last_error()
    # an odd INT4 group size over several groups is refused before anything is launched
    rc = lib.aic_hip_int4_quantize(None, 100, 7, None, None, _lib.AIC_F16, None)
    assert rc == 1 and b"even" in lib.aic_hip_last_error()
    rc = lib.aic_hip_int4_dequantize(None, None, _lib.AIC_BF16, 64, 32, None, _lib.AIC_F32, None)
    assert rc != 0 and b"scales" in lib.aic_hip_last_error()
    with pytest.raises(aic.AicError):
        _lib.call("aic_synth_uniform_ids", C.c_uint64(1), 4, 0, None)


def test_rope_tables_match_oracle_bitwise(orc):
    lib = aic.load()
    for hd in (32, 64, 128):
        S = 257
        c = np.empty((S, hd // 2), np.float32)
        s = np.empty_like(c)
        _lib.check(lib.aic_hip_rope_tables(c.ctypes.data, s.ctypes.data, S, hd, 10000.0))
        oc, os_ = orc.rope_tables(S, hd)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)


def test_synthetic_generators():
    ids, tgt = aic.batch(1234, 8, 64, 512)
    assert ids.shape == (8, 64) and ids.min() >= 0 and ids.max() < 512
    np.testing.assert_array_equal(ids[:, 1:], tgt[:, :-1])
    again, _ = aic.batch(1234, 8, 64, 512)
    np.testing.assert_array_equal(ids, again)
    z = aic.zipf_ids(7, 200000, 32000, 1.1)
    assert z.min() >= 0 and z.max() < 32000
    # Zipf(1.1): P(rank 1)/P(rank 2) = 2^1.1
    c0, c1 = np.sum(z == 0), np.sum(z == 1)
    assert abs(c0 / c1 - 2 ** 1.1) < 0.1
    w = aic.normal(5678, 1 << 20, 0.0, 0.02)
    assert abs(w.mean()) < 1e-4 and abs(w.std() - 0.02) < 2e-4
