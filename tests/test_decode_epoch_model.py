"""A host model of the one-launch decode's publish-and-observe protocol
(grimoire_amd/csrc/gemv_fused.hpp, regime 7), run over random schedules of
its work-groups, including late ones and poll time-outs.

The model follows the kernel's rules step for step:
  * a work-group reads the epoch word (epoch = word + 1, skipping 0) and the
    error word; a set error word poisons the call (NaN outputs, no
    publishing);
  * it publishes its router row tagged with the epoch, polls every router
    tag until all equal the epoch (or gives up: error word set, NaN);
  * it publishes its flag (the epoch), polls every flag likewise;
  * work-group 0 writes the epoch to the epoch word only when none of its
    polls gave up.
Kernel launches are stream-ordered: every work-group of a call exits before
the next call starts, but inside a call any work-group may start late.

Checked on every schedule: a work-group that finishes without giving up
has accepted only values written by its own call (no stale router tag or
flag is taken for current), and once any poll has given up every later call
is poisoned until the sync words are cleared (the reset entry point)."""
import random

import pytest


class Call:
    def __init__(self, ws, call_id, G, giveup):
        self.ws, self.id, self.G, self.giveup = ws, call_id, G, giveup
        self.accepted = {}            # work-group -> set of call ids it accepted
        self.outcome = {}             # work-group -> "ok" | "nan" | "poisoned"

    def wg(self, b):
        ws = self.ws
        e = (ws["epoch"] + 1) & 0xFFFFFFFF
        e = 1 if e == 0 else e
        if ws["err"]:
            self.outcome[b] = "poisoned"
            return
        yield
        ws["rtag"][b] = (e, self.id)
        yield
        bad = False
        seen = set()
        tries = 0
        while True:
            tags = list(ws["rtag"])
            if all(t[0] == e for t in tags):
                seen |= {t[1] for t in tags}
                break
            tries += 1
            if self.giveup(b, "router", tries):
                ws["err"] = 1
                bad = True
                break
            yield
        ws["flag"][b] = (e, self.id)
        yield
        tries = 0
        while True:
            fl = list(ws["flag"])
            if all(f[0] == e for f in fl):
                seen |= {f[1] for f in fl}
                break
            tries += 1
            if self.giveup(b, "flags", tries):
                ws["err"] = 1
                bad = True
                break
            yield
        if b == 0 and not bad:
            ws["epoch"] = e
        self.accepted[b] = seen
        self.outcome[b] = "nan" if bad else "ok"


def run_call(ws, call_id, G, rng, giveup, late):
    c = Call(ws, call_id, G, giveup)
    gens = {}
    pending = list(range(G))
    rng.shuffle(pending)
    # late work-groups start only after some steps of the others
    delay = {b: (rng.randrange(0, 30) if b in late else 0) for b in range(G)}
    step = 0
    while pending or gens:
        for b in list(pending):
            if delay[b] <= step:
                gens[b] = c.wg(b)
                pending.remove(b)
        if gens:
            b = rng.choice(list(gens))
            try:
                next(gens[b])
            except StopIteration:
                del gens[b]
        step += 1
        if step > 100000:
            raise AssertionError("schedule did not finish")
    return c


def fresh_ws(G):
    return {"epoch": 0, "err": 0, "rtag": [(0, -1)] * G, "flag": [(0, -1)] * G}


@pytest.mark.parametrize("seed", range(300))
def test_no_stale_value_is_taken_for_current(seed):
    rng = random.Random(seed)
    G = rng.choice([2, 3, 4])
    ws = fresh_ws(G)
    timed_out = False
    for call_id in range(6):
        late = set(rng.sample(range(G), rng.randrange(0, G)))
        limit = rng.choice([5, 40, 10 ** 6])         # poll bound in scheduler steps

        def giveup(b, what, tries, limit=limit):
            return tries > limit

        c = run_call(ws, call_id, G, rng, giveup, late)
        for b, outcome in c.outcome.items():
            if outcome == "ok":
                assert c.accepted[b] == {call_id}, (seed, call_id, b, c.accepted[b])
        if timed_out:
            assert all(o == "poisoned" for o in c.outcome.values()), (seed, call_id, c.outcome)
        if ws["err"]:
            timed_out = True
        if timed_out and rng.random() < 0.3:
            # grimoire_moe_decode_sync_reset: the sync words cleared
            ws.update(fresh_ws(G))
            timed_out = False


def test_late_group_after_a_timeout_cannot_feed_the_next_call():
    """The interleaving the protocol has to survive: work-group 1 starts
    only after work-group 0 gave up waiting for it.  Work-group 0 then must
    not advance the epoch word, the late work-group publishes under the same
    epoch as the timed-out call, and the next call is poisoned."""
    G = 2
    ws = fresh_ws(G)
    c = Call(ws, 0, G, lambda b, what, tries: b == 0 and tries > 3)
    g0 = c.wg(0)
    for _ in range(12):                 # work-group 0 alone until it gives up
        try:
            next(g0)
        except StopIteration:
            break
    assert c.outcome[0] == "nan" and ws["err"] == 1 and ws["epoch"] == 0
    for _ in c.wg(1):                   # the late work-group, same call
        pass
    c2 = run_call(ws, 1, G, random.Random(0), lambda b, w, t: t > 10 ** 6, set())
    assert all(o == "poisoned" for o in c2.outcome.values())
