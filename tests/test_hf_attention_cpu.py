"""The harness of the Hugging Face attention cases and the NumPy AttnLRP block (hf_attention_cases.py),
pinned on the CPU: the reference's own modules on its CPUBackend (oracle/_ref/libpxref.so) reproduce
the values the reference pasted from transformers 5.18.0 and from its NumPy transcription, at the
reference's tolerances. The same harness then holds MI355XBackend to them (tests/test_dropin_gpu.py)."""
import numpy as np
import pytest

import hf_attention_cases as hc
import oracle_ctypes as oc


def ref_or_skip():
    lib = oc.ref()
    if lib is None:
        pytest.skip("oracle/_ref/libpxref.so is built only where the reference sources are")
    return lib


@pytest.mark.parametrize("name", sorted(hc.CASES))
def test_reference_cpu_backend_reproduces_hf_attention_values(name):
    out, grad = hc.run_mha_case(ref_or_skip(), name)
    want_out, want_grad = hc.expected(name)
    hc.assert_matches_reference(out, want_out, name + " forward")
    hc.assert_matches_reference(grad, want_grad, name + " input gradient")


def test_reference_cpu_backend_reproduces_numpy_attnlrp_block():
    y, r = hc.run_legacy_block_case(ref_or_skip())
    v = hc.legacy_block_values()
    assert np.abs(y - np.array(v["expected_y"], np.float32)).max() <= 1e-4
    assert np.abs(r - np.array(v["expected_r_x"], np.float32)).max() <= 1e-4


def test_a_wrong_case_fails_the_harness():
    """Negative control: the Llama output moved by 0.1% (plus 1e-3) no longer passes the tolerance."""
    out, _ = hc.run_mha_case(ref_or_skip(), "llama")
    with pytest.raises(AssertionError):
        hc.assert_matches_reference(out * np.float32(1.001) + np.float32(1e-3), hc.expected("llama")[0], "perturbed")
