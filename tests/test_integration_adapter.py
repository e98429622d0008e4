"""The reference-side adapter (integration/hip_backend.cpp) compiled against
the reference's own headers and linked against libdlhip.so: the classes of
src/gpu/device.h:73-184 and src/inference/sampling/device.h:54-85 and
DeviceSequence's event type (src/inference/decoding/device.h:84-137) are
implemented on the C ABI with nothing left undefined.  Compile and link
only; skipped where the reference tree is absent."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE = "/root/reference/src"
LIB = os.path.join(ROOT, "dolittle_amd", "libdlhip.so")

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REFERENCE, "gpu", "device.h")),
                                reason="reference headers not present")


@pytest.fixture(scope="module")
def adapter(tmp_path_factory):
    if not os.path.exists(LIB):
        pytest.skip("libdlhip.so not built")
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("adapter") / "libdolittle_hip_backend.so")
    cmd = [gxx, "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror", "-fPIC", "-shared", f"-I{REFERENCE}",
           f"-I{os.path.join(ROOT, 'include')}", os.path.join(ROOT, "integration", "hip_backend.cpp"),
           f"-L{os.path.dirname(LIB)}", "-ldlhip", "-Wl,--no-undefined", "-Wl,-rpath-link,/opt/rocm/lib",
           "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def defined_symbols(path):
    r = subprocess.run(["nm", "-DC", "--defined-only", path], capture_output=True, text=True, check=True)
    return r.stdout


def test_adapter_links_with_nothing_undefined(adapter):
    assert os.path.getsize(adapter) > 0


@pytest.mark.parametrize("symbol", [
    "dolittle::gpu::Queue::upload(dolittle::gpu::DeviceRegion, dolittle::gpu::ConstHostRegion)",
    "dolittle::gpu::Queue::download(dolittle::gpu::HostRegion, dolittle::gpu::ConstDeviceRegion)",
    "dolittle::gpu::Queue::copy(dolittle::gpu::DeviceRegion, dolittle::gpu::ConstDeviceRegion)",
    "dolittle::gpu::Queue::mark()",
    "dolittle::gpu::Queue::wait(dolittle::gpu::CompletionPoint)",
    "dolittle::gpu::Queue::drain()",
    "dolittle::gpu::DeviceBuffer::size_bytes() const",
    "dolittle::gpu::HostBuffer::bytes()",
    "dolittle::gpu::hip::open_device(int)",
    "dolittle::inference::sampling::DeviceCategorical::required_bytes(unsigned long)",
    "dolittle::inference::sampling::DeviceCategorical::submit_next(dolittle::gpu::ConstDeviceRegion)",
    "dolittle::inference::sampling::DeviceCategorical::start(",
    "dolittle::inference::sampling::DeviceCategorical::result_storage() const",
    "dolittle::inference::sampling::DeviceCategorical::terminal_state() const",
    "dolittle::inference::sampling::DeviceCategorical::current_token() const",
    "dolittle::inference::hip::collect(dl_plan*, unsigned int, unsigned long, std::stop_token const&)",
])
def test_adapter_defines_the_reference_members(adapter, symbol):
    assert symbol in defined_symbols(adapter)
