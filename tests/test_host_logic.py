"""Host-side runtime logic that needs no GPU: the buffer pool's blocking and
ordering, and the transfer-strategy factory."""

import threading
import time

import pytest
import torch

from test1_amd.layer_state import LayerBufferPool


def test_pool_fifo_and_blocking():
    pool = LayerBufferPool(16, torch.bfloat16, torch.device("cpu"), 2)
    a, b = pool.acquire(), pool.acquire()
    assert a is not b and pool.available() == 0
    got = []
    t = threading.Thread(target=lambda: got.append(pool.acquire(timeout=10)))
    t.start()
    time.sleep(0.2)
    assert not got
    pool.release(a)
    t.join(5)
    assert got and got[0] is a
    with pytest.raises(TimeoutError):
        pool.acquire(timeout=0.05)
    pool.release(b)
    pool.release(a)
    assert pool.acquire() is b  # FIFO order, as the reference's deque


def test_pool_requires_two_units():
    with pytest.raises(ValueError):
        LayerBufferPool(16, torch.bfloat16, torch.device("cpu"), 1)


def test_distributed_sync_factory_single_process():
    from test1_amd import SlideFSDPConfig
    from test1_amd.distributed_sync import NoOpSync, create_distributed_sync

    s = create_distributed_sync(SlideFSDPConfig(device=torch.device("cpu")))
    assert isinstance(s, NoOpSync) and s.world_size == 1 and s.rank == 0
