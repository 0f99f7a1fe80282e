import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    # GPU tests are not skipped when no device is visible: selecting them with
    # ``-m gpu`` on a machine without an MI355X fails loudly instead.
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")
