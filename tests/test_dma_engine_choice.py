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
