"""The C-ABI library without a GPU: it loads, exports every entry point include/laya_hip.h declares,
and its host-only functions (the counter RNG, the embedding-gradient plan, argument checks that run
before any device work) behave as the reference's.

Nothing here launches a kernel or creates a context."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from laya_amd import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "laya_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(laya_\w+)\s*\(", text)))


def test_every_declared_entry_point_is_exported():
    lib = ctypes.CDLL(_native.LIB_PATH)
    names = _declared()
    assert len(names) > 70
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_every_bound_signature_is_declared():
    """The Python binding binds nothing the header does not declare."""
    declared = set(_declared())
    assert set(_native.SIGNATURES) <= declared, set(_native.SIGNATURES) - declared


def test_counter_rng_is_bit_identical_to_the_oracle():
    """Ops.Uniform / Ops.Mix (Ops.cs:227-241) on the host side of the library against the oracle's."""
    L, O = _native.lib(), oracle.lib()
    rng = np.random.default_rng(0)
    for seed, idx in zip(rng.integers(0, 2**63, 200, dtype=np.uint64), rng.integers(0, 2**40, 200, dtype=np.uint64)):
        seed, idx = int(seed), int(idx)
        u = L.laya_uniform(seed, idx)
        assert np.float32(u).tobytes() == np.float32(O.orc_uniform(seed, idx)).tobytes()
        assert 0.0 <= u < 1.0
        assert L.laya_mix(seed, idx) == O.orc_mix(seed, idx)


def test_embedding_plan_is_a_stable_sort_by_id():
    """The scatter plan of the embedding gradient (TrainableDecisionModel.cs:543-547 adds in token order):
    positions stably sorted by id, unique ids ascending, run offsets."""
    from laya_amd.ops import embedding_plan
    rng = np.random.default_rng(1)
    ids = rng.integers(0, 50, 3000).astype(np.int32)
    sorted_pos, unique_ids, offsets = embedding_plan(ids, 50)
    np.testing.assert_array_equal(sorted_pos, np.argsort(ids, kind="stable"))
    np.testing.assert_array_equal(unique_ids, np.unique(ids))
    counts = np.bincount(ids, minlength=50)[unique_ids]
    np.testing.assert_array_equal(np.diff(offsets), counts)
    assert offsets[0] == 0 and offsets[-1] == len(ids)


def test_embedding_plan_rejects_an_out_of_vocabulary_id():
    """ArgumentOutOfRangeException for a token id outside the vocabulary (TrainableDecisionModel.cs:281)."""
    from laya_amd.ops import embedding_plan
    with pytest.raises(_native.LayaOutOfRangeError):
        embedding_plan(np.array([1, 2, 50], np.int32), 50)
    with pytest.raises(_native.LayaOutOfRangeError):
        embedding_plan(np.array([-1], np.int32), 50)


def test_a_null_context_is_an_argument_error():
    """Every entry point validates its arguments before device work: a null context is refused."""
    L = _native.lib()
    assert L.laya_sync(None) == _native.ERR_ARGUMENT
    assert b"null context" in L.laya_last_error()
    assert L.laya_linear_fwd(None, None, 1, 1, None, 1, None, None, None) == _native.ERR_ARGUMENT
    assert L.laya_grad_norm_status(None) == _native.ERR_ARGUMENT


def test_status_codes_map_to_the_reference_exception_types():
    assert issubclass(_native.LayaArgumentError, ValueError)            # ArgumentException
    assert issubclass(_native.LayaOutOfRangeError, IndexError)          # ArgumentOutOfRangeException
    assert issubclass(_native.LayaMissingError, KeyError)               # InvalidDataException (missing tensor)
    assert issubclass(_native.LayaNotFiniteError, ArithmeticError)      # a non-finite gradient norm
    assert issubclass(_native.LayaMemoryError, MemoryError)
