"""Host-side logic of the runner that needs no GPU."""
import pytest

from solort_amd.runner import (DECODE_BUCKETS, PREFILL_BUCKETS, decode_qkv_splits, decode_splits, verify_bound,
                               verify_splits)


def test_decode_splits_heuristic():
    assert decode_splits(1024, 8) == 32
    assert decode_splits(128, 8) == 8
    assert decode_splits(256, 8) == 16
    assert decode_splits(512, 8) == 16
    assert decode_splits(32768, 8) == 32
    assert decode_splits(16, 8) == 1
    for bound in (2048, 4096, 8192, 16384):  # one workgroup per CU: 32 splits x 8 KV heads
        assert decode_splits(bound, 8) == 32
    assert decode_splits(65536, 8) == 64  # chunks of at most 1024 keys
    assert decode_splits(1024, 32) == 8 and decode_splits(1024, 1) == 64


def test_decode_qkv_splits_heuristic():
    for bound in (512, 1024, 2048, 4096):  # chunks of 16 to 128 keys: the fused QKV launch
        assert decode_qkv_splits(bound, 8) == 32
    for bound in (128, 256, 8192, 32768, 65536):  # elsewhere the attention's own routing
        assert decode_qkv_splits(bound, 8) == decode_splits(bound, 8)


def test_verify_bound():
    buckets = [128, 256, 512, 1024, 2048, 4096]
    # the decode bucket holding the last position, cut at the next multiple of max(128, bucket / 8)
    assert verify_bound(2052, buckets) == 2560  # 5 tokens at 2048: bucket 4096 in steps of 512
    assert verify_bound(2047, buckets) == 2048 and verify_bound(2048, buckets) == 2560
    assert verify_bound(4095, buckets) == 4096 and verify_bound(3584, buckets) == 4096
    assert verify_bound(1100, buckets) == 1280  # bucket 2048 in steps of 256
    assert verify_bound(0, buckets) == 128 and verify_bound(127, buckets) == 128 and verify_bound(128, buckets) == 256
    odd = [128, 256, 512, 1024, 2048, 3000]  # a max_len that is not a power of two
    assert verify_bound(2500, odd) == 2625 and verify_bound(2999, odd) == 3000
    for b in buckets:  # every bound holds the last position, within its bucket, at most 8 per bucket
        lo = max([x for x in buckets if x < b], default=-1)
        bounds = {verify_bound(p, buckets) for p in range(lo + 1, b)}
        assert len(bounds) <= 8 and max(bounds) == b
        assert all(p < verify_bound(p, buckets) <= b for p in range(lo + 1, b))
    with pytest.raises(RuntimeError):
        verify_bound(4096, buckets)


def test_verify_splits_heuristic():
    assert verify_splits(4096, 8) == 32 and verify_splits(2048, 8) == 16 and verify_splits(128, 8) == 1
    for bound in (8192, 16384, 32768):  # one workgroup per CU: 32 splits x 8 KV heads
        assert verify_splits(bound, 8) == 32
    assert verify_splits(65536, 8) == 64  # chunks of at most 1024 keys


def test_bucket_tables_follow_reference():
    # cuda_graph_executor.py:75-77 and :83-85
    assert DECODE_BUCKETS == (128, 256, 512, 1024, 2048, 4096)
    assert PREFILL_BUCKETS == (16, 32, 64, 128, 256, 512, 1024)
