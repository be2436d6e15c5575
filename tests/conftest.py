"""Shared pytest setup. Tests marked `gpu` need an MI355X and the built HIP library; the rest run on the CPU."""
import os, sys
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path: sys.path.insert(0, ROOT)


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs a GPU and the built libbaretile_amd.so")
