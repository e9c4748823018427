"""The v5 leaf network (engine/src/net.rs) written a second way, for the pins:
whole-tensor float64 torch over the flat blob, with the library's LayerNorm
(biased variance, eps 1e-5) and tanh-GELU, the neighbour sum as a gather from
a feature map padded with one zero hex (the form board.rs:176-193 describes
for the Rust and torch sides), and pooling as mean / amax over the hexes.

It shares no code with oracle/v5.c: the blob layout is re-derived here from
NetLayout::new's order (net.rs:272-316) and the public-row expansion from the
GPU row layout (rebel.rs:966-986) and write_public_features_raw
(rebel.rs:1144-1233).

Rounded operands: with Blob.round(kind, names), the products named in `names`
take both operands rounded to f16 or bf16 (each value first to float32, as the
float32 activations it stands for, then to nearest-even), with the products and
their sums in float64. FAST names the products the reference's fast mode runs
on tensor cores (device.rs:836-1106, 1218-1305: the card describer, the
config encoder, every trunk block's mix, out and pool-bias products, the board
and join-cache projections, the join and the readout); the stem's small
products (pile counts, hex facts, token projection, loose scalars) stay
float32.
"""
import numpy as np
import torch
import torch.nn.functional as F

TYPE, C, BLOCKS, D, POOL, CFGH, JW, JBLOCKS = 64, 96, 8, 256, 64, 128, 128, 3
FAST = frozenset({"card", "poolm", "mix", "out", "board_out", "join_p", "cfg1", "cfg_f", "cfg_g", "cfg_m", "join_b",
                  "join_w", "join_out", "values"})
JOIN_IN, HEXES, NSLOT, NTYPE, HEX_FACTS, PILES, CARD_FEATS, CFEAT, LOOSE = 129, 37, 5, 10, 6, 4, 25, 15, 15
ROW = 201


def board():
    """Neighbour table (HEXES for off-board) and location flags, from axial coordinates."""
    coords = [(x, y) for y in range(7) for x in range(7) if abs(x - 3) <= 3 and abs(y - 3) <= 3 and abs(x + y - 6) <= 3]
    index = {c: i for i, c in enumerate(coords)}
    dirs = [(1, 0), (-1, 0), (0, 1), (0, -1), (1, -1), (-1, 1)]
    nb = np.array([[index.get((x + dx, y + dy), HEXES) for dx, dy in dirs] for x, y in coords], np.int64)
    locs = [(4, 0), (6, 1), (0, 5), (2, 6), (2, 1), (3, 2), (5, 3), (1, 3), (3, 4), (4, 5)]
    loc = np.zeros(HEXES)
    for c in locs:
        loc[index[c]] = 1.0
    return nb, loc


class Blob:
    """The flat (w, b, ln) arrays cut into named float64 tensors."""

    def __init__(self, net):
        w = torch.tensor(np.asarray(net.w, np.float64))
        b = torch.tensor(np.asarray(net.b, np.float64))
        ln = torch.tensor(np.asarray(net.ln, np.float64))
        self.at_w = self.at_b = self.at_ln = 0
        self.w, self.b, self.lnv = w, b, ln
        self.q, self.fast = None, frozenset()

        def lin(i, o, bias=True):
            W = self.w[self.at_w:self.at_w + i * o].reshape(i, o)
            self.at_w += i * o
            B = None
            if bias:
                B = self.b[self.at_b:self.at_b + o]
                self.at_b += o
            return W, B

        def emb(n):
            E = self.w[self.at_w:self.at_w + n]
            self.at_w += n
            return E

        self.card = [lin(CARD_FEATS, TYPE), lin(TYPE, TYPE)]
        self.pile = lin(PILES, TYPE, False)
        self.seat = emb(2 * TYPE).reshape(2, TYPE)
        self.hex_stem = lin(HEX_FACTS, C)
        self.tok_stem = lin(TYPE, C, False)
        self.pos = emb(HEXES * C).reshape(HEXES, C)
        self.glob_stem = lin(LOOSE, C, False)
        self.blocks = [(lin(2 * C, C), lin(2 * C, C), lin(C, C)) for _ in range(BLOCKS)]
        self.board_out = lin(2 * C + LOOSE, D)
        self.cfg1 = lin(3 + TYPE, CFGH)
        self.cfg_f = lin(CFGH, D)
        self.cfg_g = lin(CFGH, POOL)
        self.cfg_m = lin(TYPE, 3 * POOL, False)
        self.join_p = lin(D, JW, False)
        self.join_b = lin(JOIN_IN, JW)
        self.join_w = [lin(JW, JW) for _ in range(JBLOCKS)]
        self.join_out = lin(JW, D)
        self.value_bias = float(self.b[self.at_b])
        self.at_b += 1
        widths = [C] * (2 * BLOCKS) + [C, CFGH] + [JW] * JBLOCKS + [JW, D]
        self.norms = []
        for width in widths:
            g = ln[self.at_ln:self.at_ln + width]
            bt = ln[self.at_ln + width:self.at_ln + 2 * width]
            self.at_ln += 2 * width
            self.norms.append((g, bt))
        assert (self.at_w, self.at_b, self.at_ln) == (len(w), len(b), len(ln))

    def round(self, kind, names=FAST):
        """Round both operands of the products in `names` to `kind` ("f16" or "bf16")."""
        dt = {"f16": torch.float16, "bf16": torch.bfloat16}[kind]
        self.q = lambda t: t.to(torch.float32).to(dt).to(torch.float64)
        self.fast = frozenset(names)
        return self

    def lin(self, name, p, x):
        """x W (+ b), the operands rounded when `name` is a rounded product."""
        W, B = p
        if self.q is not None and name in self.fast:
            x, W = self.q(x), self.q(W)
        y = x @ W
        return y if B is None else y + B


def _ln(p, x, act=True):
    g, bt = p
    y = F.layer_norm(x, (x.shape[-1],), weight=g, bias=bt, eps=1e-5)
    return F.gelu(y, approximate="tanh") if act else y


def _phys(view, t):
    return (1 - t // NSLOT if view else t // NSLOT) * NSLOT + t % NSLOT


def cards(blob, card_feat):
    """[2, NTYPE, TYPE]: view v's token t reads physical coin type _phys(v, t)."""
    cf = torch.tensor(np.asarray(card_feat, np.float64).reshape(NTYPE, CARD_FEATS))
    idx = torch.tensor([[_phys(v, t) for t in range(NTYPE)] for v in range(2)])
    x = cf[idx]
    return blob.lin("card", blob.card[1], F.gelu(blob.lin("card", blob.card[0], x), approximate="tanh"))


def expand(raw):
    """Seat-zero public inputs of GPU rows: hex facts [R, 37, 6], occupant type
    [R, 37] (-1: none), pile counts [R, 10, 4], loose scalars [R, 15]."""
    raw = np.asarray(raw, np.int64).reshape(-1, ROW)
    owner, slot, height, marker = raw[:, 0:37], raw[:, 37:74], raw[:, 74:111], raw[:, 111:148]
    _, loc = board()
    facts = np.stack([owner == 0, owner == 1, height / 5.0, marker == 0, marker == 1,
                      np.broadcast_to(loc, owner.shape)], axis=-1).astype(np.float64)
    occ = np.where((owner < 2) & (slot < NSLOT), owner * NSLOT + slot, -1)
    piles = raw[:, 148:188].reshape(-1, NTYPE, PILES) / 5.0
    loose = []
    for p in range(2):
        m = raw[:, 188 + p]
        loose += [m / 6.0, (6 - m) / 6.0, raw[:, 190 + p] / 3.0, raw[:, 192 + p] / 21.0, raw[:, 194 + p] / 21.0,
                  (raw[:, 196] == p).astype(np.float64)]
    plies = raw[:, 199] + 256 * raw[:, 200]
    loose += [plies / 256.0, (raw[:, 197] != 0).astype(np.float64), (raw[:, 198] == 0).astype(np.float64)]
    return (torch.tensor(facts), torch.tensor(occ), torch.tensor(piles, dtype=torch.float64),
            torch.tensor(np.stack(loose, axis=-1), dtype=torch.float64))


def stem(blob, raw, crd):
    """The trunk's input x [R, 37, C] and the loose scalars [R, 15] (net.rs:474-543)."""
    facts, occ, piles, loose = expand(raw)
    R = facts.shape[0]
    tok = blob.lin("pile", blob.pile, piles) + crd[0][None] + blob.seat[torch.arange(NTYPE) // NSLOT][None]
    proj = blob.lin("tok_stem", blob.tok_stem, tok)                 # [R, 10, C]
    tp = F.gelu(proj, approximate="tanh").mean(dim=1)               # [R, C]
    glob = blob.lin("glob_stem", blob.glob_stem, loose)
    occp = torch.where((occ >= 0)[..., None], proj[torch.arange(R)[:, None], occ.clamp(min=0)], torch.zeros(()))
    x = blob.lin("hex_stem", blob.hex_stem, facts) + occp + blob.pos[None] + glob[:, None] + tp[:, None]
    return x, loose


def block(blob, i, x):
    """Residual block i on x [R, 37, C] (net.rs:548-595)."""
    mix, pool, out = blob.blocks[i]
    nb = torch.tensor(board()[0])
    a = _ln(blob.norms[2 * i], x)
    pad = torch.cat([a, torch.zeros(x.shape[0], 1, C, dtype=a.dtype)], dim=1)
    neigh = pad[:, nb].sum(dim=2)                                    # [R, 37, C]
    y = blob.lin("mix", mix, torch.cat([a, neigh], dim=-1))
    gb = blob.lin("poolm", pool, torch.cat([a.mean(dim=1), a.amax(dim=1)], dim=-1))
    y = _ln(blob.norms[2 * i + 1], y + gb[:, None])
    return x + blob.lin("out", out, y)


def board_vectors(blob, raw, crd):
    """Net::board and join_cache: P [R, D], Jp [R, JW]."""
    x, loose = stem(blob, raw, crd)
    for i in range(BLOCKS):
        x = block(blob, i, x)
    x = _ln(blob.norms[2 * BLOCKS], x)
    P = blob.lin("board_out", blob.board_out, torch.cat([x.mean(dim=1), x.amax(dim=1), loose], dim=-1))
    return P, blob.lin("join_p", blob.join_p, P)


def configs(blob, phi, owner, crd):
    """Net::configs: f [n, D], g [n, POOL]."""
    phi = torch.tensor(np.asarray(phi, np.float64).reshape(-1, CFEAT))
    owner = torch.tensor(np.asarray(owner, np.int64))
    counts = phi.reshape(-1, 3, NSLOT).transpose(1, 2)                 # [n, slot, zone]
    slots = torch.cat([counts, crd[owner][:, :NSLOT]], dim=-1)         # [n, 5, 3 + TYPE]
    u = F.gelu(blob.lin("cfg1", blob.cfg1, slots), approximate="tanh").sum(dim=1)
    u = _ln(blob.norms[2 * BLOCKS + 1], u)
    f = blob.lin("cfg_f", blob.cfg_f, u)
    g = blob.lin("cfg_g", blob.cfg_g, u)
    bag = blob.lin("cfg_m", blob.cfg_m, crd).reshape(2, NTYPE, 3, POOL)             # [view, token, zone, POOL]
    g = g + torch.einsum("nkz,nkzj->nj", counts, bag[owner][:, :NSLOT])
    return f, g


def join(blob, P, Jp, pooled, player):
    """Net::join: h [R, D] from pooled [R, 2, POOL] (the player's block first)."""
    P, Jp, pooled = (torch.as_tensor(np.asarray(v, np.float64)) for v in (P, Jp, pooled))
    seat = torch.full((P.shape[0], 1), -1.0 if player == 0 else 1.0, dtype=torch.float64)
    z = Jp + blob.lin("join_b", blob.join_b, torch.cat([pooled[:, 0], pooled[:, 1], seat], dim=-1))
    for i in range(JBLOCKS):
        z = z + blob.lin("join_w", blob.join_w[i], _ln(blob.norms[2 * BLOCKS + 2 + i], z))
    z = _ln(blob.norms[2 * BLOCKS + 2 + JBLOCKS], z)
    return _ln(blob.norms[2 * BLOCKS + 3 + JBLOCKS], P + blob.lin("join_out", blob.join_out, z), act=False)


def values(blob, f, h):
    """Net::values for every (row of h, config of f): [R, n]."""
    h, f = torch.as_tensor(np.asarray(h, np.float64)), torch.as_tensor(np.asarray(f, np.float64))
    return blob.lin("values", (f.T, None), h) + blob.value_bias
