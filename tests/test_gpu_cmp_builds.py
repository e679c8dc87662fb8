"""Two independently loaded copies of this build agree bit for bit on every hot entry point
(stblarge_amd/cmp_builds.py): the kernels are deterministic run to run, and the comparison tool that
guards performance work works."""

import pytest

from stblarge_amd import _lib, cmp_builds

pytestmark = pytest.mark.gpu


def test_build_against_itself(gpu):
    _lib.load()
    assert cmp_builds.compare(_lib.LIB_PATH, _lib.LIB_PATH, seeds=1) == []
