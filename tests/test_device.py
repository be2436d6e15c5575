"""Device claims on the host (docs/api.md:43-45, test/test_device.py:69): one opener at a time holds a GPU, in this
process or another. No GPU needed: the claim is host logic (a registry and an flock), checked on a GPU index no test
opens."""
import fcntl, gc, os

from baretile_amd import pci

N = 61  # a GPU index for the claim alone; nothing here asks HIP for it


def test_one_claim_per_process_released_on_drop():
  a = pci._take(N)
  assert a is not None and pci._take(N) is None
  del a
  gc.collect()
  b = pci._take(N)
  assert b is not None
  del b


def test_claim_held_by_another_open_file_is_refused():
  # flock locks belong to an open file, so a second open of the lock file stands in for another process
  fd = os.open(pci.lock_path(N), os.O_RDWR | os.O_CREAT, 0o666)
  try:
    fcntl.flock(fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
    assert pci._take(N) is None
  finally:
    os.close(fd)
  c = pci._take(N)
  assert c is not None
  del c
