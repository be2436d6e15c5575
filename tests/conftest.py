"""Shared pytest setup. Tests marked `gpu` need an MI355X and the built HIP library; the rest run on the CPU."""
import os, sys
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path: sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path: sys.path.insert(0, HERE)


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs a GPU and the built libbaretile_amd.so")


@pytest.fixture(scope="session")
def chip():
  """The first GPU, as a Chip. A GPU test that finds none fails: it never falls back to the CPU."""
  from baretile_amd import pci
  from baretile_amd.chip import Chip
  return Chip(pci.open_device())


@pytest.fixture
def rt(chip):
  from baretile_amd.runtime import Runtime
  r = Runtime(chip)
  yield r
  r.close()
