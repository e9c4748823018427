"""Textbook vanilla CFR over world states, for pinning the oracle.

Nothing here knows about public belief states or the reverse tables: a world
state is (public node, config of player 0, config of player 1), an
information set is (public node, the acting player's own config), chance is a
real chance player whose probability enters the counterfactual reach, and the
prior over root configs enters each player's own reach. The pattern is the
reference's exhaustive check (engine/tests/rebel_solver.rs:68-162): run
vanilla CFR from every root config pair, average the traverser-0 root value
over the second half of the run. Only terminal leaves are supported (no value
network), so the whole game is inside the subgame.
"""
from __future__ import annotations

import numpy as np

NONE = 0xFFFFFFFF


class Game:
    """Read-only view of one decoded WCJ8 job (tests/wcj8.py)."""

    def __init__(self, j: dict):
        self.j = j
        self.term = {int(n): float(u) for n, u in zip(j["term_leaves"], j["terminal_utility"])}
        if len(j["leaf_rows"]):
            raise ValueError("brute-force CFR needs a tree of terminal leaves only")

    def nc(self, node, p):
        o = self.j["cfg_off"]
        return int(o[2 * node + p + 1] - o[2 * node + p])

    def kind(self, node):
        return int(self.j["node_kind"][node])

    def player(self, node):
        return int(self.j["node_player"][node])

    def cells(self, node, c):
        """Legal cells of the actor's config c: (child node, successor config or NONE)."""
        j = self.j
        row = int(j["legal_row_of"][node]) + c
        lo, hi = int(j["legal_off"][row]), int(j["legal_off"][row + 1])
        return [(int(j["legal_child"][g]), int(j["legal_trans"][g])) for g in range(lo, hi)]

    def outcomes(self, node, c):
        """Chance outcomes of the drawer's config c: (successor config, probability)."""
        j = self.j
        d0, rb = int(j["draw_off"][node]), int(j["draw_row_off"][node])
        lo, hi = int(j["draw_row_start"][rb + c]), int(j["draw_row_start"][rb + c + 1])
        return [(int(j["draw_to"][d0 + x]), float(j["draw_p"][d0 + x])) for x in range(lo, hi)]

    def child(self, node):
        return int(self.j["node_child"][self.j["node_child_start"][node]])


def _regret_match(r):
    pos = np.maximum(r, 0.0)
    s = pos.sum()
    return pos / s if s > 0 else np.full(len(r), 1.0 / len(r))


def _cfr(g, tab, node, cfg, reach, chance, trav):
    kind = g.kind(node)
    if kind == 2:
        u = g.term[node]
        return u if g.player(node) == trav else -u
    me = g.player(node)
    if kind == 1:
        v = 0.0
        for to, pr in g.outcomes(node, cfg[me]):
            nxt = list(cfg)
            nxt[me] = to
            v += pr * _cfr(g, tab, g.child(node), nxt, reach, chance * pr, trav)
        return v
    key = (node, cfg[me])
    cells = g.cells(node, cfg[me])
    reg = tab["regret"].setdefault(key, np.zeros(len(cells)))
    sigma = _regret_match(reg)
    util = np.zeros(len(cells))
    for a, (child, trans) in enumerate(cells):
        if trans == NONE:
            util[a] = 0.0  # the world leaves the tracked supports: value 0
            continue
        nxt = list(cfg)
        nxt[me] = trans
        r = list(reach)
        r[me] *= sigma[a]
        util[a] = _cfr(g, tab, child, nxt, r, chance, trav)
    node_util = float(sigma @ util)
    if me == trav:
        cf = reach[1 - trav] * chance
        reg += cf * (util - node_util)
        st = tab["strat"].setdefault(key, np.zeros(len(cells)))
        st += reach[trav] * sigma
    return node_util


def game_value(job: dict, iters: int = 200) -> float:
    """Value for player 0 under the root prior, averaged over the second half."""
    g = Game(job)
    bel = [np.asarray(job["root"][0], np.float64), np.asarray(job["root"][1], np.float64)]
    tab = {"regret": {}, "strat": {}}
    value, count = 0.0, 0
    for it in range(iters):
        trav = it % 2
        total = 0.0
        for c0 in range(len(bel[0])):
            for c1 in range(len(bel[1])):
                pr = [bel[0][c0], bel[1][c1]]
                v = _cfr(g, tab, 0, [c0, c1], pr, 1.0, trav)
                if trav == 0:
                    total += pr[0] * pr[1] * v
        if trav == 0 and 2 * it >= iters:
            value += total
            count += 1
    return value / count
