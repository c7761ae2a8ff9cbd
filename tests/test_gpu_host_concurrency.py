"""Under the gpu mark: the host metadata under concurrent threads (test_host_meta_concurrency.py).

These tests call only host entry points, so they also run without a GPU; this
module collects them again under the gpu mark, so that the library the GPU run
loads is the one they check.
"""
import pytest

from test_host_meta_concurrency import test_shipped_library_aba_and_churn, test_shipped_library_concurrent_cow_forks  # noqa: F401

pytestmark = pytest.mark.gpu
