"""Every route of the dispatch trees is exercised by the GPU suite.

A route ends in one instantiation of a kernel template, so the check is: every
kernel instantiation compiled into libnq_hip.so (its host-side kernel handles)
appears in profiles/gpu_test_kernel_coverage.txt, the kernel trace of
`pytest tests -m gpu` (written by tests/route_coverage.py), with the first test
that launched it. CPU only: it reads the library's symbol table and the
committed trace summary."""
import os
import shutil

import pytest

import route_coverage as rc

# instantiation -> why no GPU test launches it
NOT_LAUNCHED = {}


@pytest.mark.skipif(not shutil.which("nm") or not shutil.which("c++filt"), reason="binutils not available")
def test_every_kernel_instantiation_is_launched_by_a_gpu_test():
    lib = rc.library_kernels()
    assert len(lib) > 100
    cov = rc.read_summary()
    missing = sorted(k for k in lib if k not in cov and k not in NOT_LAUNCHED)
    assert not missing, "kernel instantiations no GPU test launches:\n" + "\n".join(missing)
    stale = sorted(k for k in cov if k not in lib)
    assert not stale, "the coverage summary names kernels the library no longer has:\n" + "\n".join(stale)
    for k in sorted(lib):
        if k in cov:
            print(f"{k}  <-  {cov[k][1]}")


def test_summary_is_from_the_gpu_suite():
    assert os.path.exists(rc.SUMMARY)
    cov = rc.read_summary()
    tests = {t for _, t in cov.values()}
    assert all(t.startswith("tests/") for t in tests), [t for t in tests if not t.startswith("tests/")][:5]
