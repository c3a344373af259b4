"""The drop-in claim, checked where the reference sources are present (this container, not the
GPU box): MI355XBackend compiles against the reference's own DeviceBackend header, overriding
every virtual with the reference's exact signature."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"


@pytest.mark.skipif(not os.path.isfile(os.path.join(REF, "include", "pulsatrix", "device_backend.hpp")),
                    reason="reference sources not present")
def test_mi355x_backend_compiles_against_reference_device_backend():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "dropin-check", "REF=" + REF],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
