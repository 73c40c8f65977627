"""The device image generator (synth.image_device) computes the same bytes as synth.image: the
same fp64 operations in the same order, run here with torch on the CPU over several row blocks."""
import numpy as np
import pytest

from odie_amd import synth


@pytest.mark.parametrize('width,height,rows', [(97, 61, 16), (200, 150, 1000), (640, 333, 100)])
def test_device_image_equals_numpy_image(width, height, rows):
    expected = synth.image(3, width, height)
    got = synth.image_device(3, width, height, device='cpu', rows=rows).numpy()
    assert got.dtype == np.uint8 and got.shape == (height, width, 3)
    assert np.array_equal(got, expected)
