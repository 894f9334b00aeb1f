"""Shared pytest setup: the `gpu` marker and import paths."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

# The compiled reference reads PK_THREADS once, on its first pk_pool() call.
os.environ.setdefault("PK_THREADS", str(min(os.cpu_count() or 1, 16)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
