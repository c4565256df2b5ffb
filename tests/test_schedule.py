"""Pins ``oracle.step_schedule`` (the unit schedule of one training step)
without retyping it, two ways:

1. An event model of the reference's control flow: the forward records the
   autograd nodes the reference creates (slide_fsdp.py:535-637: the embedding,
   then per decoder a ``PreLayerFunction``, the checkpointed layer under
   ``SlidingCheckpoint`` and a ``PostLayerFunction``, then the output unit),
   runs their forward actions, and the backward replays the recorded nodes in
   reverse with their backward actions (slide_fsdp.py:404-409, 432-464;
   sliding_checkpoint.py:51-131).  Loads go through a residency flag that
   makes a load of a unit still on the device a no-op, as
   ``to_device_async`` does (layer_state.py:286-287).  The model is built
   from node types and state, not from a loop over the schedule; the two must
   agree for every L = 1..8, every set of resident decoders, with and without
   checkpoint offload, and in both orders of the first two loads.
2. Invariants read off the reference's structure, checked on every schedule:
   forward loads, the grads flag of the output unit, backward reloads and
   their place before the next gradient offload, one offload per unit in
   reverse order, the checkpoint packs and where each prefetch falls.

Mistakes planted in the oracle (the last decoder reloaded, a prefetch two
units ahead, the output unit's grads flag dropped, a checkpoint prefetched a
unit late, the embedding's reload missing) must each be caught by both.
"""

import itertools
from collections import deque

import pytest

import oracle


# ---------------------------------------------------------------------------
# 1. event model of the reference's step
# ---------------------------------------------------------------------------

class RefStepModel:
    """Autograd nodes and residency flags of one reference training step.

    Units: 0 embedding, 1..L decoders, L+1 output (norm + lm_head).
    ``resident`` decoders keep their device buffer from their forward to their
    backward, as the reference's last decoder does (its ``PostLayerFunction``
    is called with ``is_last_layer=True`` and skips the offload,
    slide_fsdp.py:399-400, 631)."""

    def __init__(self, L, act_offload=True, resident=(), first_decoder_first=False):
        self.L = L
        self.act = act_offload
        self.resident = set(resident)
        self.first_decoder_first = first_decoder_first
        self.on_device = set()      # units whose _current_gpu_cache is set
        self.events = []
        self.tape = []              # nodes recorded by the forward, in order
        self.prefetched = deque()   # checkpoint prefetch FIFO (sliding_checkpoint.py:7)

    # --- LayerRuntimeState, reduced to what orders events
    def to_device_async(self, u, is_backward):
        if u in self.on_device:     # layer_state.py:286-287
            return
        self.on_device.add(u)
        self.events.append(("h2d", u, is_backward))

    def offload_forward(self, u):
        self.on_device.discard(u)   # layer_state.py:383-393: views back to host, unit released

    def offload_backward(self, u):
        self.events.append(("d2h", u))   # slide_fsdp.py:450-464 -> layer_state.py:339-399
        self.on_device.discard(u)

    # --- nodes
    def post_forward(self, u, is_last_layer):
        if not is_last_layer and u not in self.resident:
            self.offload_forward(u)
        self.tape.append(("post", u))

    def pre_forward(self, u, next_u):
        if next_u is not None:      # slide_fsdp.py:370-373
            self.to_device_async(next_u, is_backward=next_u == self.L + 1)
        self.tape.append(("pre", u))

    def checkpointed_layer(self, u):
        d = u - 1                   # SlidingCheckpoint.layer_idx (sliding_checkpoint.py:26)
        last = u == self.L
        if self.act and not last:   # pack hook: every decoder but the last (:58-59)
            self.events.append(("act_d2h", u))
        self.tape.append(("ckpt", u, d, last))

    def plain_layer(self, u):
        self.tape.append(("layer", u))

    # --- the step
    def forward(self):
        L = self.L
        first = [0, 1]              # slide_fsdp.py:536-541
        if self.first_decoder_first:
            first.reverse()
        for u in first:
            self.to_device_async(u, False)
        self.plain_layer(0)
        self.post_forward(0, False)
        for u in range(1, L + 1):
            self.pre_forward(u, u + 1)
            self.checkpointed_layer(u)
            self.post_forward(u, u == L)
        self.pre_forward(L + 1, None)
        self.plain_layer(L + 1)
        self.post_forward(L + 1, True)

    def backward(self):
        for node in reversed(self.tape):
            kind = node[0]
            if kind == "post":      # PostLayerFunction.backward -> _on_pre_backward
                u = node[1]
                if u - 1 >= 0:
                    self.to_device_async(u - 1, True)
            elif kind == "ckpt":    # recompute: the first unpack prefetches decoder d-1
                _, u, d, last = node
                if self.act and d - 1 >= 0:
                    self.events.append(("act_h2d", u - 1))
                    self.prefetched.append(u - 1)
                if self.act and not last:
                    # the unpack of a non-last decoder is served from the FIFO head
                    assert self.prefetched and self.prefetched.popleft() == u, "checkpoint FIFO out of order"
                self.offload_backward(u)
            elif kind == "layer":
                self.offload_backward(node[1])
            # "pre": PreLayerFunction.backward is a no-op (slide_fsdp.py:383-386)
        assert not self.prefetched, "a prefetched checkpoint was never used"

    def run(self):
        self.forward()
        self.backward()
        return self.events


def model_schedule(L, act, resident, first_decoder_first):
    return RefStepModel(L, act, resident, first_decoder_first).run()


# ---------------------------------------------------------------------------
# 2. invariants from the reference's structure
# ---------------------------------------------------------------------------

def violations(s, L, act, resident, first_decoder_first):
    """Broken invariants of schedule ``s`` (empty when it holds them all)."""
    bad = []
    out = L + 1
    d2h_pos = {}
    for k, e in enumerate(s):
        if e[0] == "d2h":
            if e[1] in d2h_pos:
                bad.append(f"d2h({e[1]}) twice")
            d2h_pos[e[1]] = k
    first_d2h = min(d2h_pos.values()) if d2h_pos else len(s)
    fwd, bwd = s[:first_d2h], s[first_d2h:]

    # d2h: every unit once, output first, embedding last (slide_fsdp.py:450-464)
    if [e[1] for e in s if e[0] == "d2h"] != list(range(out, -1, -1)):
        bad.append("d2h order is not L+1..0")

    # forward loads: units 0..L+1, each once; only the output unit with grads
    # (slide_fsdp.py:372-373), the first two up front in either order
    loads = [e for e in fwd if e[0] == "h2d"]
    units = [e[1] for e in loads]
    head = [1, 0] if first_decoder_first else [0, 1]
    if units != head + list(range(2, out + 1)):
        bad.append(f"forward loads {units}")
    for e in loads:
        if e[2] != (e[1] == out):
            bad.append(f"forward load of unit {e[1]} with grads={e[2]}")
    if any(e[0] in ("act_h2d",) for e in fwd):
        bad.append("checkpoint prefetch in the forward")

    # one ahead of use: PreLayerFunction(u) loads unit u+1 and runs before
    # decoder u's checkpointed forward, whose pack hook marks the decoder, so
    # the forward's events between two packs are exactly one load
    if act:
        segs, cur = [], []
        for e in fwd:
            if e[0] == "act_d2h":
                segs.append(cur)
                cur = []
            else:
                cur.append(e[:2])
        segs.append(cur)
        want = [[("h2d", u) for u in head] + [("h2d", 2)]] + [[("h2d", u + 2)] for u in range(1, L)]
        if segs != want:
            bad.append(f"forward loads not one ahead: {segs}")

    # checkpoint packs: decoders 1..L-1 in order (the last keeps its input on
    # the device, sliding_checkpoint.py:58-59)
    packs = [e[1] for e in s if e[0] == "act_d2h"]
    if packs != (list(range(1, L)) if act else []):
        bad.append(f"checkpoint packs {packs}")

    # backward reloads: units {0..L-1} minus resident, strictly decreasing, all
    # with grads; each before the offload of the unit above it
    # (slide_fsdp.py:432-448; layer_state.py:286-287 makes a resident unit's
    # reload a no-op)
    reloads = [e for e in bwd if e[0] == "h2d"]
    ru = [e[1] for e in reloads]
    want = [u for u in range(L - 1, -1, -1) if u not in resident]
    if ru != want:
        bad.append(f"backward reloads {ru}, expected {want}")
    if not all(e[2] for e in reloads):
        bad.append("a backward reload without grads")
    bpos = {(e[0], e[1]): k for k, e in enumerate(bwd)}
    for u in ru:
        a, b = bpos.get(("d2h", u + 2)), bpos.get(("d2h", u + 1))
        if a is None or b is None or not (a < bpos[("h2d", u)] < b):
            bad.append(f"reload of unit {u} not between d2h({u + 2}) and d2h({u + 1})")

    # checkpoint prefetches: decoder j's input (j = L-1..1) after d2h(j+2) and
    # before d2h(j+1): issued by decoder j+1's first unpack, one layer ahead
    # (sliding_checkpoint.py:88-108)
    pre = [e[1] for e in s if e[0] == "act_h2d"]
    if pre != (list(range(L - 1, 0, -1)) if act else []):
        bad.append(f"checkpoint prefetches {pre}")
    for j in pre:
        k = bpos.get(("act_h2d", j))
        a, b = bpos.get(("d2h", j + 2)), bpos.get(("d2h", j + 1))
        if k is None or a is None or b is None or not (a < k < b):
            bad.append(f"prefetch of decoder {j} not between d2h({j + 2}) and d2h({j + 1})")
    return bad


def cases(max_L=8):
    for L in range(1, max_L + 1):
        decoders = list(range(1, L))   # the last decoder is resident in any case
        for r in range(len(decoders) + 1):
            for resident in itertools.combinations(decoders, r):
                for act in (True, False):
                    yield L, act, resident


# ---------------------------------------------------------------------------
# tests
# ---------------------------------------------------------------------------

def test_oracle_matches_reference_event_model():
    n = 0
    for L, act, resident in cases():
        for ffirst in (False, True):
            exp = model_schedule(L, act, resident, ffirst)
            got = oracle.step_schedule(L, act_offload=act, first_decoder_first=ffirst, resident_units=resident)
            assert got == exp, (L, act, resident, ffirst)
            n += 1
    assert n == 2 * 2 * sum(2 ** (L - 1) for L in range(1, 9))   # 1,020 schedules


def test_oracle_holds_the_invariants():
    for L, act, resident in cases():
        for ffirst in (False, True):
            s = oracle.step_schedule(L, act_offload=act, first_decoder_first=ffirst, resident_units=resident)
            assert violations(s, L, act, resident, ffirst) == [], (L, act, resident, ffirst)


def test_model_of_the_reference_by_hand_l2():
    """L = 2, checkpoints offloaded, reference order, worked through the
    reference's code by hand."""
    assert model_schedule(2, True, (), False) == [
        ("h2d", 0, False), ("h2d", 1, False),            # slide_fsdp.py:536-541
        ("h2d", 2, False), ("act_d2h", 1),               # PreLayer(1) prefetches 2; decoder 1 packs
        ("h2d", 3, True),                                # PreLayer(2) prefetches the output unit with grads
        ("d2h", 3),                                      # output unit's backward
        ("h2d", 1, True), ("act_h2d", 1), ("d2h", 2),    # PostLayer(2).bwd reloads 1; 2's unpack prefetches 1
        ("h2d", 0, True), ("d2h", 1),                    # PostLayer(1).bwd reloads the embedding
        ("d2h", 0),
    ]


# Mistakes planted in the oracle: each mutant must be rejected by both checks.
def _last_decoder_reloaded(L, act, resident, ffirst):
    s = oracle.step_schedule(L, act, ffirst, resident)
    k = s.index(("d2h", L + 1))
    return s[:k + 1] + [("h2d", L, True)] + s[k + 1:]


def _prefetch_two_ahead(L, act, resident, ffirst):
    """Each PreLayerFunction(u) loads unit u+2 instead of u+1: unit 2 joins the
    loads made up front and PreLayerFunction(L) loads nothing."""
    s = oracle.step_schedule(L, act, ffirst, resident)
    end = s.index(("d2h", L + 1))
    idx = [k for k in range(end) if s[k][0] == "h2d"]
    loads = [s[k] for k in idx]
    out, j = [], 0
    for k, e in enumerate(s):
        if k in idx:
            if j < 2:
                out.append(e)
                if j == 1:
                    out.append(loads[2])
            elif j + 1 < len(loads):
                out.append(loads[j + 1])
            j += 1
        else:
            out.append(e)
    return out


def _grads_flag_dropped(L, act, resident, ffirst):
    s = oracle.step_schedule(L, act, ffirst, resident)
    return [("h2d", L + 1, False) if e == ("h2d", L + 1, True) else e for e in s]


def _checkpoint_prefetched_late(L, act, resident, ffirst):
    """Each decoder's checkpoint fetched when its own backward starts, not one layer ahead."""
    s = oracle.step_schedule(L, act, ffirst, resident)
    out = [e for e in s if e[0] != "act_h2d"]
    for j in range(L - 1, 0, -1):
        k = out.index(("d2h", j + 1))
        out.insert(k + 1, ("act_h2d", j))
    return out


def _embedding_reload_missing(L, act, resident, ffirst):
    s = oracle.step_schedule(L, act, ffirst, resident)
    return [e for e in s if e != ("h2d", 0, True)]


# (mutant, applies to (L, act)): a prefetch distance or a checkpoint prefetch
# is only visible where the forward or backward has checkpoint events.
MUTANTS = [
    (_last_decoder_reloaded, lambda L, act: True),
    (_prefetch_two_ahead, lambda L, act: act and L >= 2),
    (_grads_flag_dropped, lambda L, act: True),
    (_checkpoint_prefetched_late, lambda L, act: act and L >= 2),
    (_embedding_reload_missing, lambda L, act: True),
]


@pytest.mark.parametrize("mutant,applies", MUTANTS, ids=[m.__name__.strip("_") for m, _ in MUTANTS])
def test_planted_mistakes_are_caught(mutant, applies):
    seen = 0
    for L, act, resident in cases(6):
        if not applies(L, act):
            continue
        for ffirst in (False, True):
            bad = mutant(L, act, resident, ffirst)
            assert bad != model_schedule(L, act, resident, ffirst), (mutant.__name__, L, act, resident)
            assert violations(bad, L, act, resident, ffirst), (mutant.__name__, L, act, resident)
            seen += 1
    assert seen > 0
