"""Shared pytest setup: the `gpu` marker, import paths, and a build when nothing is built."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

if not (os.path.exists(os.path.join(ROOT, "large_model_amd", "libqmsg.so")) and
        os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so"))):
    import __graft_entry__
    __graft_entry__.build()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libqmsg.so")
