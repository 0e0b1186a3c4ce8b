"""The kernels' quotient forms against IEEE binary32 division, over every input of their domains.

The reference divides in IEEE binary32 (engine/kernels.c:84 the mean of squares, :98-99 the block
scale and its reciprocal, :395 SiLU).  The HIP kernels form those quotients from a reciprocal
estimate and fused residual corrections on domains where they are exact, with the IEEE division
as the fallback elsewhere; q4hip_check_division runs each form over all of its inputs (2^31 or
2^32 bit patterns) on the device and counts results whose bits differ from the IEEE quotient's.
"""
import pytest

pytestmark = pytest.mark.gpu


def test_every_quotient_form_is_exact():
    import q4hip
    counts = q4hip.check_division()
    print(counts, flush=True)
    assert set(counts) == set(q4hip.DIVISION_FORMS)
    assert all(v == 0 for v in counts.values()), counts
