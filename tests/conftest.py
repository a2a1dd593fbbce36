"""Pytest configuration: repo root on sys.path and the `gpu` marker.

Tests marked `gpu` run the HIP kernels through the C ABI and are skipped on a
machine without a GPU; everything else runs on the CPU.

When a GPU test dies in native code (an abort from the HIP runtime, a GPU
fault), the log must still say where: each GPU test's id is written to the
terminal as it starts, and Python's fault handler dumps only the crashing
thread, whose innermost frames then fit in a truncated log tail.
"""

import faulthandler
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

_GPU_IDS: set = set()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.hookimpl(trylast=True)
def pytest_sessionstart(session):
    # After pytest's own fault-handler plugin: same file, current thread only.
    fd = None
    try:
        from _pytest.faulthandler import fault_handler_stderr_fd_key

        fd = session.config.stash.get(fault_handler_stderr_fd_key, None)
    except ImportError:
        pass
    faulthandler.enable(file=fd if fd is not None else sys.__stderr__, all_threads=False)


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        _GPU_IDS.update(item.nodeid for item in items if "gpu" in item.keywords)
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tests run on an MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_runtest_logstart(nodeid, location):
    if nodeid in _GPU_IDS:
        sys.__stderr__.write(f"\n[gpu test] {nodeid}\n")
        sys.__stderr__.flush()
