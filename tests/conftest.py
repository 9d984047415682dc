import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "vla-to-npu_amd"
for p in (str(PKG_ROOT), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")
