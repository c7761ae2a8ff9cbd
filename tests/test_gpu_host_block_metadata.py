"""Under the gpu mark: the free stack, refcounts and BlockTable against the reference's KATs and the oracle (test_block_metadata.py).

These tests call only host entry points, so they also run without a GPU; this
module collects them again under the gpu mark, so that the library the GPU run
loads is the one they check.
"""
import pytest

from test_block_metadata import *  # noqa: F401,F403  (the tests and their fixtures)

pytestmark = pytest.mark.gpu
