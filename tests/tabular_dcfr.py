"""Discounted CFR iterate by iterate over world states, for pinning the oracle's
trajectory (not only its fixed point).

Nothing here shares the oracle's form. The oracle backs belief vectors up a
public tree in reverse node order; this module evaluates world states: the
expected utility V(node, c0, c1) of a public node with both players' private
configs fixed, by memoised recursion, and each player's own reach factor
(prior x own strategy x own draws) by a forward pass over the public tree.
The counterfactual action value of the traverser's information state
(node, c) is then

    q(cell) = sum_{c'} reach_opp(node, c') * V(child, trans(c), c')

(engine/src/search.rs:1654-1803 computes the same quantity as a vector over
c; the traverser's own draw probabilities enter through V, not through the
weight), and the regret update is the published one: discounted CFR (Brown and
Sandholm, AAAI 2019) with alternating updates, the predictive term of
PCFR+ (Farina et al., AAAI 2021) and the reference's EPS floor in regret
matching. The schedule is what the reference fixes and what this module pins:

- player p's m-th own update (m = 1, 2, ...) discounts p's accumulated regrets
  by m^alpha / (m^alpha + 1) where positive and m^beta / (m^beta + 1) where
  not, before adding the new instantaneous regret (search.rs:1659-1667,
  1755-1761);
- the average-strategy sum of p's nodes is discounted by (m / (m + 1))^gamma,
  then the new strategy weighted by p's reach under that new strategy is added
  (search.rs:1777-1779, 1805-1835);
- the sums start from one reach-weighted uniform strategy of both players
  (search.rs:852-870), and the strategy of a player who never updated is the
  literal uniform one (search.rs:899-937).

Only terminal leaves are supported (no value network). Everything is float64.
"""
from __future__ import annotations

import math

import numpy as np

NONE = 0xFFFFFFFF
EPS = 1e-6


def factor(m: float, p: float) -> float:
    """m^p / (m^p + 1), with p = +inf (keep) and -inf (discard) as limits."""
    if math.isinf(p):
        return 1.0 if p > 0 else 0.0
    x = m ** p
    return x / (x + 1.0)


class Tree:
    """The public tree of one decoded WCJ8 job (tests/wcj8.py), terminal leaves only."""

    def __init__(self, j: dict):
        if len(j["leaf_rows"]):
            raise ValueError("the tabular solver needs a tree of terminal leaves only")
        self.j = j
        self.n = int(j["nodes"])
        self.term = {int(n): float(u) for n, u in zip(j["term_leaves"], j["terminal_utility"])}
        self.kind = [int(k) for k in j["node_kind"]]
        self.player = [int(p) for p in j["node_player"]]
        self.ncells = int(j["legal_off"][-1])

    def nc(self, node, p):
        o = self.j["cfg_off"]
        return int(o[2 * node + p + 1] - o[2 * node + p])

    def row(self, node, c):
        """Global cell indices of the actor's config c, with (child, trans) each."""
        j = self.j
        r = int(j["legal_row_of"][node]) + c
        return [(g, int(j["legal_child"][g]), int(j["legal_trans"][g]))
                for g in range(int(j["legal_off"][r]), int(j["legal_off"][r + 1]))]

    def draws(self, node, c):
        j = self.j
        d0, rb = int(j["draw_off"][node]), int(j["draw_row_off"][node])
        lo, hi = int(j["draw_row_start"][rb + c]), int(j["draw_row_start"][rb + c + 1])
        return [(int(j["draw_to"][d0 + x]), float(j["draw_p"][d0 + x])) for x in range(lo, hi)]

    def children(self, node):
        j = self.j
        return [int(j["node_child"][k]) for k in range(int(j["node_child_start"][node]),
                                                       int(j["node_child_start"][node + 1]))]


def own_reach(t: Tree, sigma: np.ndarray, prior, p: int):
    """reach[node][c]: prior x p's own strategy x p's own draws, over p's configs."""
    reach = [np.zeros(t.nc(i, p)) for i in range(t.n)]
    reach[0][:] = np.asarray(prior, np.float64)
    for i in range(t.n):  # children follow their parents in node order
        k = t.kind[i]
        if k == 2:
            continue
        r = reach[i]
        if k == 1 and t.player[i] == p:
            ch = t.children(i)[0]
            for c in range(len(r)):
                for to, pr in t.draws(i, c):
                    reach[ch][to] += r[c] * pr
        elif k == 0 and t.player[i] == p:
            for c in range(len(r)):
                for g, ch, tr in t.row(i, c):
                    if tr != NONE:
                        reach[ch][tr] += r[c] * sigma[g]
        else:  # the other player moves or draws: p's config index is kept
            for ch in t.children(i):
                reach[ch] += r
    return reach


def world_values(t: Tree, sigma: np.ndarray, p: int):
    """V(node, c0, c1) for player p: expected terminal utility under sigma and both players' draws."""
    memo = {}

    def V(i, c0, c1):
        key = (i, c0, c1)
        if key in memo:
            return memo[key]
        k, me = t.kind[i], t.player[i]
        cfg = [c0, c1]
        if k == 2:
            u = t.term[i]
            v = u if me == p else -u
        elif k == 1:
            ch = t.children(i)[0]
            v = 0.0
            for to, pr in t.draws(i, cfg[me]):
                nxt = list(cfg)
                nxt[me] = to
                v += pr * V(ch, *nxt)
        else:
            v = 0.0
            for g, ch, tr in t.row(i, cfg[me]):
                if tr == NONE:  # the world leaves the tracked supports: value 0
                    continue
                nxt = list(cfg)
                nxt[me] = tr
                v += sigma[g] * V(ch, *nxt)
        memo[key] = v
        return v

    return V


class Solver:
    def __init__(self, j: dict):
        self.t = Tree(j)
        self.j = j
        t = self.t
        self.prior = [np.asarray(j["root"][0], np.float64), np.asarray(j["root"][1], np.float64)]
        self.alpha, self.beta, self.gamma, self.predict = (float(j["alpha"]), float(j["beta"]), float(j["gamma"]),
                                                           float(j["predict"]))
        self.sigma = np.zeros(t.ncells)
        for i in range(t.n):
            if t.kind[i] == 0:
                for c in range(t.nc(i, t.player[i])):
                    row = t.row(i, c)
                    for g, _, _ in row:
                        self.sigma[g] = 1.0 / len(row)
        self.regret = np.zeros(t.ncells)
        self.sum = np.zeros(t.ncells)
        self.steps = [0, 0]
        for p in (0, 1):
            self._add_average(p)

    def decision_rows(self, p):
        t = self.t
        for i in range(t.n):
            if t.kind[i] == 0 and t.player[i] == p:
                for c in range(t.nc(i, p)):
                    yield i, c, t.row(i, c)

    def _add_average(self, p):
        reach = own_reach(self.t, self.sigma, self.prior[p], p)
        for i, c, row in self.decision_rows(p):
            for g, _, _ in row:
                self.sum[g] += reach[i][c] * self.sigma[g]

    def step(self, p):
        t = self.t
        m = self.steps[p] + 1.0
        da, db, dg = factor(m, self.alpha), factor(m, self.beta), (m / (m + 1.0)) ** self.gamma
        opp = own_reach(t, self.sigma, self.prior[1 - p], 1 - p)
        V = world_values(t, self.sigma, p)
        new_sigma = self.sigma.copy()
        for i, c, row in self.decision_rows(p):
            q = np.zeros(len(row))
            for a, (g, ch, tr) in enumerate(row):
                if tr == NONE:
                    continue
                for co in range(t.nc(i, 1 - p)):
                    w = opp[i][co]
                    q[a] += w * (V(ch, tr, co) if p == 0 else V(ch, co, tr))
            base = float(sum(self.sigma[g] * q[a] for a, (g, _, _) in enumerate(row)))
            pos = np.zeros(len(row))
            for a, (g, _, _) in enumerate(row):
                delta = q[a] - base
                old = self.regret[g]
                r = old * (da if old > 0 else db) + delta
                self.regret[g] = r
                pos[a] = max(r + self.predict * delta, EPS)
            pos /= pos.sum()
            for a, (g, _, _) in enumerate(row):
                new_sigma[g] = pos[a]
        self.sigma = new_sigma
        for i, c, row in self.decision_rows(p):
            for g, _, _ in row:
                self.sum[g] *= dg
        self._add_average(p)
        self.steps[p] += 1

    def average(self):
        """The final average strategy per cell (a player who never updated: the current one)."""
        out = self.sigma.copy()
        for p in (0, 1):
            if self.steps[p] == 0:
                continue
            for i, c, row in self.decision_rows(p):
                s = sum(self.sum[g] for g, _, _ in row)
                for g, _, _ in row:
                    out[g] = self.sum[g] / s if s > 0 else 1.0 / len(row)
        return out

    def root_values(self, strategy, beliefs):
        """Per-config root values of both players under `strategy` from root beliefs (b0, b1):
        player p's value of config c = sum_{c'} b_{1-p}(c') V_p(0, c, c')."""
        t = self.t
        out = []
        for p in (0, 1):
            V = world_values(t, strategy, p)
            b = np.asarray(beliefs[1 - p], np.float64)
            out.append(np.array([sum(b[co] * (V(0, c, co) if p == 0 else V(0, co, c)) for co in range(len(b)))
                                 for c in range(t.nc(0, p))]))
        return np.concatenate(out)


def solve(j: dict, iters: int | None = None):
    """Run `iters` alternating iterations (the job's own count by default):
    (average strategy per cell, root values per carried root [nroots, n0 + n1])."""
    s = Solver(j)
    for it in range(int(j["iters"]) if iters is None else iters):
        s.step(it % 2)
    avg = s.average()
    roots = [s.root_values(avg, pair) for pair in j["carried"]]
    return avg, (np.stack(roots) if roots else np.zeros((0, 0)))
