"""Under the gpu mark: the XXH3 prefix hash against its vectors and the prefix map rules (test_prefix_cache.py).

These tests call only host entry points, so they also run without a GPU; this
module collects them again under the gpu mark, so that the library the GPU run
loads is the one they check.
"""
import pytest

from test_prefix_cache import *  # noqa: F401,F403  (the tests and their fixtures)

pytestmark = pytest.mark.gpu
