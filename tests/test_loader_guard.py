"""The external-data guard of the weight-pack loader
(mmnb_check_external_ref), on the reference's own cases
(test/parser_robustness_test.dart:65-97).  Pure host code: no GPU needed."""
import pytest

from onnx_runtime_dart_amd.model import check_external_ref


@pytest.mark.parametrize("loc", ["../../etc/passwd", "/etc/passwd", "weights/../../../secret",
                                 r"C:\Windows\x", ""])
def test_path_traversal_and_absolute_paths_reject(loc):
    with pytest.raises(ValueError):
        check_external_ref(loc, 0, 0, 1 << 20)


@pytest.mark.parametrize("off,ln", [(-1, 10), (0, -5), (0, 1 << 40), (990, 20)])
def test_out_of_bounds_ranges_reject(off, ln):
    with pytest.raises(ValueError):
        check_external_ref("w.bin", off, ln, 1000)


def test_valid_in_bounds_relative_reference_passes():
    check_external_ref("weights.bin", 100, 400, 1000)
    check_external_ref("sub/weights.bin", 0, 1000, 1000)
