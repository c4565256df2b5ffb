"""The SDMA engine choice of the gradient copies (sf_dma_choose_engines, the
pure part of sf_dma_copy_d2h), on the CPU: engines that another client holds
(busy with no copy of ours pending) are replaced by free ones among 0-3, and
in mode 2 by twice as many free engines from 4 up when none of 0-3 is free."""

import pytest

E = lambda *engines: sum(1 << e for e in engines)  # noqa: E731
ALL = 0xFFFF


@pytest.fixture(scope="module")
def choose():
    from test1_amd import _native
    return _native.hip().sf_dma_choose_engines


def test_nothing_held_keeps_the_selection(choose):
    assert choose(E(2, 3), ALL, 0, 2) == E(2, 3)
    # busy with our own copies only: not held
    assert choose(E(2, 3), ALL & ~E(2, 3), E(2, 3), 2) == E(2, 3)
    assert choose(E(2, 3), ALL & ~E(0, 1, 2, 3), E(2, 3), 2) == E(2, 3)


def test_held_engine_replaced_by_a_free_one_among_0_to_3(choose):
    # engine 2 busy and none of our copies on it: held (a HIP copy waiting on an event)
    assert choose(E(2, 3), ALL & ~E(2), 0, 1) == E(0, 3)
    assert choose(E(2, 3), ALL & ~E(0, 2), 0, 2) == E(1, 3)
    # both held: the two free ones among 0-3
    assert choose(E(2, 3), ALL & ~E(2, 3), 0, 1) == E(0, 1)
    # engine 3 busy with ours, engine 2 held, 0 busy (HIP): 1 replaces 2
    assert choose(E(2, 3), ALL & ~E(0, 2, 3), E(3), 2) == E(1, 3)


def test_all_fast_engines_held(choose):
    held_0_3 = ALL & ~E(0, 1, 2, 3)
    # mode 1 keeps to 0-3: nothing better than the selection itself
    assert choose(E(2, 3), held_0_3, 0, 1) == E(2, 3)
    # mode 2: twice as many free engines from 4 up
    assert choose(E(2, 3), held_0_3, 0, 2) == E(4, 5, 6, 7)
    assert choose(E(2, 3), E(9, 12), 0, 2) == E(9, 12)
    # none free anywhere: the selection
    assert choose(E(2, 3), 0, 0, 2) == E(2, 3)
    # one fast engine usable: no slow ones added
    assert choose(E(2, 3), held_0_3 | E(3), 0, 2) == E(3)


def test_off_and_degenerate_selections(choose):
    assert choose(E(2, 3), ALL & ~E(2, 3), 0, 0) == E(2, 3)   # mode 0: routing off
    assert choose(0, 0, 0, 2) == 0                            # runtime's own choice stays
    assert choose(E(2) | (1 << 20), ALL & ~E(2), 0, 1) == E(0)  # bits past engine 15 ignored


def test_choice_invariants_over_random_masks(choose):
    """For random selections, free masks and our-copy masks: mode 0 and any
    selection without a held engine come back unchanged; otherwise the
    choice is the selection (nothing better free) or a set with no held
    engine, made of the selection's unheld engines plus free engines (among
    0-3, or from 4 up in mode 2 when none of 0-3 could be had), never larger
    than twice the selection."""
    import random
    rng = random.Random(7)
    for _ in range(20000):
        preferred = rng.getrandbits(16) & rng.getrandbits(16)
        avail = rng.getrandbits(16)
        ours = rng.getrandbits(16) & ~avail & 0xFFFF
        mode = rng.randrange(3)
        got = choose(preferred, avail, ours, mode)
        held = ~avail & ~ours & 0xFFFF
        if mode == 0 or preferred == 0 or not (preferred & held):
            assert got == preferred
            continue
        if got == preferred:
            continue   # nothing usable: keep the selection
        assert not (got & held), (preferred, avail, ours, mode, got)
        extra = got & ~preferred
        assert not (extra & ~avail), "an added engine must be free"
        fast = extra & 0xF
        assert bin(got).count("1") <= 2 * bin(preferred).count("1")
        if extra & ~0xF:
            assert mode == 2 and not (got & preferred & ~held) and not fast, "slow engines only when no fast one"


# ---------------------------------------------------------------------------
# SF_DMA_AVOID_HELD: parsed strictly, and any mode but 0 refused for training
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("value,mode", [(None, 0), ("", 0), ("  ", 0), ("0", 0), ("1", 1), ("2", 2), (" 2 ", 2)])
def test_avoid_held_env_values(value, mode):
    from test1_amd import kernels
    assert kernels.avoid_held_from_env(value) == mode


@pytest.mark.parametrize("value", ["3", "-1", "yes", "1.5", "0x1"])
def test_avoid_held_env_rejects_other_values(value):
    from test1_amd import kernels
    with pytest.raises(ValueError, match="SF_DMA_AVOID_HELD"):
        kernels.avoid_held_from_env(value)


class _InitStub:
    """The sf_dma_* entry points dma_init calls, recording them."""

    def __init__(self):
        self.calls = []

    def sf_dma_init(self, dev):
        self.calls.append(("init", dev))
        return 0

    def sf_dma_set_engines(self, mask):
        self.calls.append(("engines", mask))
        return 0

    def sf_dma_set_avoid_held(self, mode):
        self.calls.append(("avoid_held", mode))
        return 0


@pytest.mark.parametrize("value", ["1", "2"])
def test_dma_init_refuses_routing(monkeypatch, value):
    """Mode 1 used to be skipped silently and mode 2 turned routing on; both
    now raise before the library is touched."""
    from test1_amd import _native, kernels
    stub = _InitStub()
    monkeypatch.setattr(_native, "hip", lambda: stub)
    monkeypatch.setattr(kernels, "_dma_ready", set())
    monkeypatch.setenv("SF_DMA_AVOID_HELD", value)
    with pytest.raises(RuntimeError, match="routing"):
        kernels.dma_init(__import__("torch").device("cuda", 0))
    assert stub.calls == []


@pytest.mark.parametrize("value", [None, "", "0"])
def test_dma_init_with_routing_off(monkeypatch, value):
    from test1_amd import _native, kernels
    stub = _InitStub()
    monkeypatch.setattr(_native, "hip", lambda: stub)
    monkeypatch.setattr(kernels, "_dma_ready", set())
    if value is None:
        monkeypatch.delenv("SF_DMA_AVOID_HELD", raising=False)
    else:
        monkeypatch.setenv("SF_DMA_AVOID_HELD", value)
    monkeypatch.setenv("SF_DMA_ENGINES", "4,5")
    kernels.dma_init(__import__("torch").device("cuda", 3))
    assert stub.calls == [("init", 3), ("engines", (1 << 4) | (1 << 5))]
    kernels.require_routing_off()


def test_runtime_refuses_routing_set_through_the_api(monkeypatch):
    from test1_amd import _native, kernels
    stub = _InitStub()
    monkeypatch.setattr(_native, "hip", lambda: stub)
    monkeypatch.delenv("SF_DMA_AVOID_HELD", raising=False)
    monkeypatch.setattr(kernels, "_avoid_held_mode", 0)
    kernels.dma_set_avoid_held(2)
    try:
        with pytest.raises(RuntimeError, match="routing"):
            kernels.require_routing_off()
    finally:
        kernels.dma_set_avoid_held(0)
    kernels.require_routing_off()


@pytest.mark.parametrize("value,engines", [(None, None), ("", None), (" ", None), ("3", [3]), ("2,3", [2, 3]),
                                           (" 2, 3 ", [2, 3]), ("0,15", [0, 15])])
def test_engines_from_env(value, engines):
    from test1_amd import kernels
    assert kernels.engines_from_env(value) == engines


@pytest.mark.parametrize("value", ["16", "-1", "x", "2,,3", "2;3", "3.0"])
def test_engines_from_env_rejects_other_values(value):
    from test1_amd import kernels
    with pytest.raises(ValueError, match="SF_DMA_ENGINES"):
        kernels.engines_from_env(value)


def test_dma_init_refuses_a_bad_engine_list(monkeypatch):
    from test1_amd import _native, kernels
    stub = _InitStub()
    monkeypatch.setattr(_native, "hip", lambda: stub)
    monkeypatch.setattr(kernels, "_dma_ready", set())
    monkeypatch.delenv("SF_DMA_AVOID_HELD", raising=False)
    monkeypatch.setenv("SF_DMA_ENGINES", "16")
    with pytest.raises(ValueError, match="SF_DMA_ENGINES"):
        kernels.dma_init(__import__("torch").device("cuda", 0))
    assert stub.calls == []
