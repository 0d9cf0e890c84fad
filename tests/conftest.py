import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libgqa.so")


def pytest_collection_modifyitems(config, items):
    """When GPU tests are selected, bring up torch's HIP runtime before any libgqa context
    exists, so every GPU test sees the same initialisation order (torch first, then the
    library) whichever test uses torch first."""
    if not any(item.get_closest_marker("gpu") for item in items):
        return
    try:
        import torch
    except ImportError:
        return
    if torch.cuda.is_available():
        torch.cuda.init()
        torch.empty(1, device="cuda")
