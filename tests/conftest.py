"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` tests run anywhere (oracle pins, host logic, ABI exports);
`-m gpu` tests need an MI355X and call the HIP kernels through the C ABI.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "nano-vllm-kv-optimizer_amd")
for p in (PKG_ROOT, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libnanokv.so")
