"""Host-side validation of the NLA device objects' Python mirror
(dolittle_amd/interventions.py), which raises the reference's exception
classes before any device work (injection/device.h:29-47,
steering/device.h:30-68).  No GPU: a stand-in buffer carries only a size,
and a stand-in device refuses allocation, so every case below must fail in
validation."""
import math

import pytest

from dolittle_amd.interventions import DeviceDirection, DeviceInjection, DeviceIntervention, Region


class Buffer:
    def __init__(self, nbytes):
        self.nbytes = nbytes

    def ptr(self, offset=0):
        raise AssertionError("no device access expected")


class NoDevice:
    def allocate(self, *args):
        raise AssertionError("validation must fail before allocation")


@pytest.mark.parametrize("scale", [0.0, -1.0, math.inf, math.nan])
def test_injection_scale(scale):
    with pytest.raises(ValueError):
        DeviceInjection(NoDevice(), None, Region(Buffer(8192), 0, 8192), "bfloat16", "bfloat16", 4096, scale)


def test_injection_region_and_types():
    dev = NoDevice()
    with pytest.raises(ValueError):  # region shorter than width * 2
        DeviceInjection(dev, None, Region(Buffer(8192), 0, 4096), "bfloat16", "bfloat16", 4096, 150.0)
    with pytest.raises(ValueError):  # region past the buffer
        DeviceInjection(dev, None, Region(Buffer(8192), 2, 8192), "bfloat16", "bfloat16", 4096, 150.0)
    with pytest.raises(ValueError):  # misaligned FP32 source
        DeviceInjection(dev, None, Region(Buffer(1 << 20), 2, 16384), "float32", "bfloat16", 4096, 150.0)
    with pytest.raises(ValueError):
        DeviceInjection(dev, None, Region(Buffer(8192), 0, 8192), "float16", "bfloat16", 4096, 150.0)


def test_direction_and_intervention_validation():
    dev = NoDevice()
    good = Region(Buffer(8192), 0, 8192)
    with pytest.raises(ValueError):
        DeviceDirection(dev, None, good, Region(Buffer(8192), 0, 4096), "bfloat16", 4096)
    with pytest.raises(ValueError):
        DeviceDirection(dev, None, good, good, "int8", 4096)
    direction = Region(Buffer(16384), 0, 16384)
    for strength in (-0.5, math.nan, math.inf):
        with pytest.raises(ValueError):
            DeviceIntervention(dev, None, direction, 4096, 3, strength, "bfloat16")
    with pytest.raises(ValueError):  # direction region of the wrong width
        DeviceIntervention(dev, None, Region(Buffer(16384), 0, 8192), 4096, 3, 1.0, "bfloat16")
