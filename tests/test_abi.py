"""The C-ABI library loads and exports every entry point declared in include/*.h."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from summa_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sm_\w+)\s*\(", re.M)


def declared():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        names += DECL.findall(h.read_text())
    return names


def test_header_declares_entry_points():
    names = declared()
    assert "sm_ce_rows" in names and "sm_grpo_loss" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libsumma_amd.so not built (python -m summa_amd.build)")
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(raw, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    assert set(_lib.SIGNATURES) == set(declared())


def test_host_only_calls():
    L = _lib.lib()
    assert L.sm_version() >= 1
    assert L.sm_grpo_flags_message(0) is None
    assert L.sm_grpo_flags_message(1 << 3).decode() == \
        "GRPO active_mask must contain only binary zero/one values"


def test_argument_errors_are_reported_not_raised():
    L = _lib.lib()
    # invalid clip epsilon is rejected before any device work
    st = L.sm_grpo_loss(1, 1, 1, None, None, 1, 2, 1, 1.5, 1e-6, 0.0, None, None, None, None, None)
    assert st == -1
    assert L.sm_last_error().decode() == "GRPO clip_epsilon must be finite and in (0, 1)"
    st = L.sm_ce_rows(1, 1, 1, 4, 8, 9, None, None, None, 1.0, None, None, None)
    assert st == -1 and b"logical vocabulary 9" in L.sm_last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(top_k=0), "top_k must be >= 1 (got 0)"),
    (dict(temperature=float("nan")), "temperature must not be NaN"),
    (dict(repetition_penalty=0.5), "repetition_penalty must be finite and >= 1 (got 0.5)"),
    (dict(repetition_penalty=float("inf")), "repetition_penalty must be finite and >= 1 (got inf)"),
    (dict(top_p=0.0), "rollout top_p must be finite and in (0, 1]"),
    (dict(top_p=1.5), "rollout top_p must be finite and in (0, 1]"),
    (dict(eos_token=10), "eos_token 10 is outside the model vocabulary of 10 entries"),
])
def test_sampling_options_rejected_with_reference_messages(kw, msg):
    """generate.rs:68-84 and RolloutSampling::validate (posttrain.rs:372-386):
    rejected before any device work."""
    import ctypes
    from summa_amd.sampling import SamplingConfig
    L = _lib.lib()
    sc = SamplingConfig(**kw).c()
    st = L.sm_sample_ex(1, 1, 10, 10, ctypes.addressof(sc), 0, 0, None, 0, None, None, 1, 1,
                        None, 1, None, None)
    assert st == -1
    assert L.sm_last_error().decode() == msg


def test_rollout_sampling_validate_messages():
    from summa_amd.sampling import RolloutSampling
    RolloutSampling().validate()
    for kw, msg in [(dict(max_new_tokens=0), "max_new_tokens must be in 1..=1048576"),
                    (dict(temperature=0.0), "rollout temperature must be finite and positive"),
                    (dict(top_p=float("nan")), "rollout top_p must be finite and in (0, 1]")]:
        with pytest.raises(ValueError, match=msg.replace("(", r"\(").replace(")", r"\)")
                           .replace("[", r"\[").replace("]", r"\]").replace(".", r"\.")):
            RolloutSampling(**kw).validate()


def test_gemv_multi_plan_host_checks():
    """sm_q4_gemv_multi_plan validates every job and fills first_block and the
    block -> job table on the host (no device memory is touched)."""
    import numpy as np
    L = _lib.lib()
    jobs = (_lib.GemvJob * 3)()
    for i, (n, k) in enumerate([(40, 256), (16, 128), (1, 512)]):
        jobs[i] = _lib.GemvJob(4096, 8192, 16384, 32768, n, k, _lib.SM_EPI_STORE_F32, -1)
    total = L.sm_q4_gemv_multi_plan(ctypes.byref(jobs), 3, None)
    assert total == 3 + 1 + 1
    table = np.full(total, -1, dtype=np.int32)
    L.sm_q4_gemv_multi_plan(ctypes.byref(jobs), 3, table.ctypes.data_as(ctypes.c_void_p))
    assert [j.first_block for j in jobs] == [0, 3, 4]
    assert table.tolist() == [0, 0, 0, 1, 2]
    jobs[1].K = 100
    assert L.sm_q4_gemv_multi_plan(ctypes.byref(jobs), 3, None) == -1
    assert b"job 1" in L.sm_last_error()
    jobs[1].K = 128
    jobs[2].epilogue = _lib.SM_EPI_SWIGLU_F16
    assert L.sm_q4_gemv_multi_plan(ctypes.byref(jobs), 3, None) == -1
    assert b"job 2" in L.sm_last_error()


def test_linear_cross_entropy_host_checks():
    """sm_linear_cross_entropy rejects bad arguments with the reference's
    messages (linear_cross_entropy/mod.rs:66-69, reference.rs:21-30) before
    any device work; the workspace query refuses bad shapes."""
    L = _lib.lib()
    assert L.sm_linear_cross_entropy_workspace_bytes(0, 8, 16, 4, 0) == -1
    assert L.sm_linear_cross_entropy_workspace_bytes(4, 8, 16, 4, 1) > 4 * 16 * 4
    ws = 1 << 20
    st = L.sm_linear_cross_entropy(16, 16, None, 16, 4, 8, 16, 16, 0, 0, 16, None, ws, 1 << 20,
                                   None)
    assert st == -1 and L.sm_last_error().decode() == \
        "linear cross-entropy chunk size must be positive"
    st = L.sm_linear_cross_entropy(16, 16, None, 16, 0, 8, 16, 16, 2, 0, 16, None, ws, 1 << 20,
                                   None)
    assert st == -1 and L.sm_last_error().decode() == \
        "linear cross-entropy requires at least one token"
    st = L.sm_linear_cross_entropy_backward(16, 16, None, 16, 16, 4, 8, 16, 20, 2, 0, 16, 16,
                                            None, ws, 1 << 20, None)
    assert st == -1 and L.sm_last_error().decode() == "logical vocabulary 20 must be in 1..=16"
    st = L.sm_linear_cross_entropy(16, 16, None, 16, 4, 8, 16, 16, 2, 0, 16, None, ws, 100, None)
    assert st == -1 and b"workspace holds 100 bytes" in L.sm_last_error()


def test_grouped_linear_and_row_permute_host_checks():
    """The grouped expert projections and the route permutation reject bad
    arguments before any device work: counts that do not cover the routes or
    hold a negative entry (grouped_linear_inner takes per-expert row counts,
    summa-llm/src/model/grouped_linear.rs:23-60), a missing scratch, an
    unsupported dtype and an output that aliases the input."""
    import numpy as np

    L = _lib.lib()
    dummy = 1 << 20  # never dereferenced: each call fails its checks first
    for counts, msg in (([2, 3], b"cover the input (5 != 6)"),
                        ([7, -1], b"negative count for expert 1")):
        c = np.asarray(counts, dtype=np.int64)
        st = L.sm_grouped_linear(dummy, dummy, c.ctypes.data, 2, 6, 4, 3, dummy, None)
        assert st == -1 and msg in L.sm_last_error()
        st = L.sm_grouped_linear_backward(dummy, dummy, dummy, c.ctypes.data, 2, 6, 4, 3, dummy,
                                          dummy, None)
        assert st == -1 and msg in L.sm_last_error()
    st = L.sm_grouped_linear(dummy, dummy, None, 2, 6, 4, 3, dummy, None)
    assert st == -1 and b"null counts" in L.sm_last_error()
    c = np.asarray([6, 0], dtype=np.int64)
    st = L.sm_grouped_swiglu_mlp_backward(dummy, dummy, dummy, c.ctypes.data, 2, 6, 4, 5, 3,
                                          dummy, dummy, dummy, dummy, dummy, dummy, None, None)
    assert st == -1 and b"null buffer" in L.sm_last_error()
    st = L.sm_row_permute(dummy, 7, 4, 8, dummy, dummy + 4096, None)
    assert st == -1 and b"dtype must be" in L.sm_last_error()
    st = L.sm_row_permute(dummy, 0, 4, 8, dummy + 64, dummy, None)
    assert st == -1 and b"must not alias" in L.sm_last_error()
    assert L.sm_row_permute(dummy, 0, 0, 8, dummy + 64, dummy + 4096, None) == 0
