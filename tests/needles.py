"""Closed-form "needle" cases for the attention kernels (not collected by pytest).

Every (sequence, kv head) group gets three planted keys, all multiples of one
random +-1 vector u[kv head] (shared by every sequence, so a key read from the
wrong sequence or page would also dominate):

  key 0            a * u      floor needle, score ~ 45 nats
  key p (moving)   2a * u     the needle, score ~ 90 nats
  key Lk (paged)   4a * u     poison one past the last key, score ~ 181 nats

and every query row of the group is a * u plus N(0, 0.25^2) noise; all other
keys and values are N(0, 1), whose scores stay below ~10 nats.  The softmax
is then one-hot to far below bf16 precision, so the exact output is known
without an oracle: a query row t of a sequence with Lq queries and Lk keys
sees key j iff j <= t + Lk - Lq, hence

    out[t, h] = V[p]   if p <= t + Lk - Lq
                V[0]   otherwise,

bit for bit (the probabilities of the needle row are exactly 1 and everything
else contributes < 1e-12 relative).  A kernel that drops a key at a tile,
page, chunk or wave-split edge, shifts the causal diagonal, or reads the key
past the end returns another row of V, an O(1) error.  Moving p over every
64-key tile edge, 32-key chunk edge and page edge of every group over a run
of calls places a needle on every point where a kernel can cut a context.
"""
from __future__ import annotations

import torch

A = 2.0          # |q| scale: needle score 2 * A^2 * D * D^-0.5 = 90.5 nats at D = 128
NOISE = 0.25     # per-row query noise, so the rows are not all identical


def interesting_positions(lk: int, step: int, block_size: int, lq: int = 1) -> list[int]:
    """Key positions in [1, lk) where a kernel can cut a context: both sides of
    every `step`-key edge and every page edge, the first keys, the last keys
    and the first new key (lk - lq)."""
    s = {1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 255, 256, 257, lk - 2, lk - 1,
         lk - lq - 1, lk - lq, lk - lq + 1}
    for e in range(step, lk, step):
        s.update((e - 1, e))
    for e in range(block_size, lk, block_size):
        s.update((e - 1, e, e + 1))
    return sorted(p for p in s if 1 <= p < lk)


class NeedleCase:
    """q / K / V with planted needles for `lens_q` query rows over `lens_k`
    keys per sequence.  Paged (block_size > 0): private pages per sequence,
    enough for key Lk (the poison).  Dense (block_size == 0): key j of
    sequence s is row cu_k[s] + j of [Tk, Hkv, D] tensors (no poison: the row
    after a sequence is the next sequence's floor needle, which the shared u
    would make visible if it were read)."""

    def __init__(self, seed, lens_q, lens_k, block_size=256, hq=16, hkv=8, d=128,
                 device="cuda", dtype=torch.bfloat16):
        assert all(lk >= 2 for lk in lens_k) and len(lens_q) == len(lens_k)
        self.lens_q, self.lens_k = list(lens_q), list(lens_k)
        self.bs, self.hq, self.hkv, self.d = block_size, hq, hkv, d
        self.g = hq // hkv
        self.device = torch.device(device)
        self.scale = d ** -0.5
        b = len(lens_k)
        cpu = torch.Generator().manual_seed(seed)
        gen = torch.Generator(device=self.device).manual_seed(seed)
        bf = dtype
        cu_q = [0]
        for n in lens_q:
            cu_q.append(cu_q[-1] + n)
        cu_k = [0]
        for n in lens_k:
            cu_k.append(cu_k[-1] + n)
        self.cu_q = torch.tensor(cu_q, dtype=torch.int32, device=self.device)
        self.cu_k = torch.tensor(cu_k, dtype=torch.int32, device=self.device)
        if block_size:
            pages = [lk // block_size + 1 for lk in lens_k]        # keys 0 .. lk
            nb = sum(pages) + 2
            perm = torch.randperm(nb, generator=cpu).tolist()
            bt = torch.full((b, max(pages)), -1, dtype=torch.int32)
            nxt = 0
            for i, p in enumerate(pages):
                bt[i, :p] = torch.tensor(perm[nxt:nxt + p], dtype=torch.int32)
                nxt += p
            self.block_tables = bt.to(self.device)
            shape = (nb, block_size, hkv, d)
        else:
            self.block_tables = None
            shape = (cu_k[-1], hkv, d)
        self.k = torch.randn(*shape, generator=gen, device=self.device).to(bf)
        self.v = torch.randn(*shape, generator=gen, device=self.device).to(bf)
        u = torch.randn(hkv, d, generator=gen, device=self.device).sign()
        self.u = torch.where(u == 0, torch.ones_like(u), u)
        tq = cu_q[-1]
        uq = self.u.repeat_interleave(self.g, 0)
        self.q = (A * uq[None] + NOISE * torch.randn(tq, hq, d, generator=gen,
                                                        device=self.device)).to(bf)
        # per query row: its sequence and its index inside the sequence
        seq = torch.repeat_interleave(torch.arange(b), torch.tensor(lens_q))
        self.row_seq = seq.to(self.device)
        self.row_t = (torch.arange(tq) - torch.tensor(cu_q[:-1])[seq]).to(self.device)
        self.diag = torch.tensor([lk - lq for lq, lk in zip(lens_q, lens_k)],
                                 device=self.device)
        self.heads = torch.arange(hkv, device=self.device)
        zero = torch.zeros(b, hkv, dtype=torch.long, device=self.device)
        kf = self.k.view(-1, hkv, d)
        kf[self.slots(zero), self.heads] = (A * self.u).to(bf)[None]
        if block_size:
            lk_t = torch.tensor(lens_k, device=self.device)[:, None].expand(b, hkv)
            kf[self.slots(lk_t), self.heads] = (4 * A * self.u).to(bf)[None]
        self.dtype = bf

    def slots(self, pos: torch.Tensor) -> torch.Tensor:
        """Row of key pos[s, h] of sequence s in the flat [rows, Hkv, D] view."""
        s = torch.arange(pos.shape[0], device=self.device)[:, None]
        if self.bs:
            page = torch.gather(self.block_tables.long(), 1, pos // self.bs)
            return page * self.bs + pos % self.bs
        return self.cu_k.long()[:-1][:, None] + pos + 0 * s

    def plant(self, pos: torch.Tensor):
        """Put the needle at key pos[s, h] of every group; returns what to
        pass to restore()."""
        kf = self.k.view(-1, self.hkv, self.d)
        sl = self.slots(pos)
        saved = kf[sl, self.heads].clone()
        kf[sl, self.heads] = (2 * A * self.u).to(self.dtype)[None]
        return sl, saved

    def restore(self, planted) -> None:
        sl, saved = planted
        self.k.view(-1, self.hkv, self.d)[sl, self.heads] = saved

    def expected(self, pos: torch.Tensor) -> torch.Tensor:
        """[Tq, Hq, D] bf16: V[p] for rows that see key p, else V[0]."""
        vf = self.v.view(-1, self.hkv, self.d)
        vn = vf[self.slots(pos), self.heads]                                   # [B, Hkv, D]
        v0 = vf[self.slots(torch.zeros_like(pos)), self.heads]
        sees = pos[self.row_seq] <= (self.row_t + self.diag[self.row_seq])[:, None]
        e = torch.where(sees[..., None], vn[self.row_seq], v0[self.row_seq])   # [Tq, Hkv, D]
        return e.repeat_interleave(self.g, 1)

    def position_schedule(self, step: int) -> list[torch.Tensor]:
        """Calls that together put the needle of every group on each of its
        sequence's interesting positions (heads rotate, so one call covers
        several positions of a sequence)."""
        lists = [interesting_positions(lk, step, self.bs or (1 << 30), lq)
                 for lq, lk in zip(self.lens_q, self.lens_k)]
        n_calls = max(len(x) for x in lists)
        calls = []
        for c in range(n_calls):
            p = [[lst[(c + 5 * h) % len(lst)] for h in range(self.hkv)] for lst in lists]
            calls.append(torch.tensor(p, dtype=torch.long, device=self.device))
        return calls


def mismatches(out: torch.Tensor, exp: torch.Tensor) -> torch.Tensor:
    """Per row and head: 1 where out differs from exp by more than one bf16
    ulp (the expected rows are exact; the ulp covers the < 1e-12 relative
    contribution of every other key; an f16 ulp is smaller still)."""
    o, e = out.float(), exp.float()
    bad = (o - e).abs() > e.abs() * 2.0 ** -8 + 1e-6
    return bad.any(dim=-1)


def run_schedule(case: NeedleCase, call, step: int, what: str) -> int:
    """Plant, call, compare for every call of the schedule; returns the number
    of calls.  `call(case)` returns the kernel output [Tq, Hq, D]."""
    from gpu_utils import say
    calls = case.position_schedule(step)
    say(f"needles {what}: {len(calls)} calls")
    fails = []
    for pos in calls:
        planted = case.plant(pos)
        out = call(case).reshape(-1, case.hq, case.d)
        fails.append(mismatches(out, case.expected(pos)).sum())
        case.restore(planted)
    fails = torch.stack(fails).cpu()
    if int(fails.sum()):
        i = int(torch.nonzero(fails)[0])
        pos = calls[i]
        planted = case.plant(pos)
        out = call(case).reshape(-1, case.hq, case.d)
        bad = mismatches(out, case.expected(pos))
        case.restore(planted)
        r, h = [int(x) for x in torch.nonzero(bad)[0]]
        s = int(case.row_seq[r])
        raise AssertionError(
            f"{what}: call {i}: {int(fails[i])} rows wrong; first: row {r} (sequence {s}, query "
            f"{int(case.row_t[r])} of {case.lens_q[s]}, keys {case.lens_k[s]}), head {h}, "
            f"needle at key {int(pos[s, h // case.g])}")
    return len(calls)
