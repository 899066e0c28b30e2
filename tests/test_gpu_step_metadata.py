"""Device-side step metadata (nvk_prefill_metadata / nvk_decode_metadata)
against the host builders that restate the reference's loops
(model_runner.py:123-188): every tensor of the Context must be identical."""
import random

import pytest
import torch

from oracle import step_metadata as metadata
from nanovllm_amd.engine.device_metadata import prepare_decode_device, prepare_prefill_device
from oracle.sequence import Sequence
from nanovllm_amd.utils.context import get_context, reset_context
from tests.gpu_utils import say

pytestmark = pytest.mark.gpu


def _snapshot():
    c = get_context()
    out = {}
    for f in ("is_prefill", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k",
              "slot_mapping", "context_lens", "block_tables"):
        v = getattr(c, f)
        out[f] = v.cpu() if isinstance(v, torch.Tensor) else v
    reset_context()
    return out


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        x, y = a[k], b[k]
        if isinstance(x, torch.Tensor) or isinstance(y, torch.Tensor):
            assert isinstance(x, torch.Tensor) and isinstance(y, torch.Tensor), k
            assert x.dtype == y.dtype and x.shape == y.shape and torch.equal(x, y), k
        else:
            assert x == y, k


def _prefill_seqs(rng, n, bs, pool, cached_max, new_max, with_tables=True):
    pages = list(range(pool))
    rng.shuffle(pages)
    nxt = 0
    seqs = []
    for _ in range(n):
        c = rng.randint(0, cached_max)
        m = rng.randint(1, new_max)
        need = (c + m + bs - 1) // bs
        table = pages[nxt:nxt + need] if with_tables else []
        nxt += need
        seqs.append(Sequence([rng.randint(0, 150000) for _ in range(c + m)], block_table=table,
                             num_cached_tokens=c, num_scheduled_tokens=m))
    return seqs


@pytest.mark.parametrize("n,bs,cached_max,new_max", [(1, 256, 0, 700), (7, 256, 1000, 600),
                                                     (33, 16, 90, 70), (64, 256, 1536, 1024)])
def test_prefill_metadata_equals_host_builder(n, bs, cached_max, new_max):
    say(f"prefill metadata n={n} bs={bs}")
    rng = random.Random(n * 7 + bs)
    seqs = _prefill_seqs(rng, n, bs, pool=n * ((cached_max + new_max) // bs + 2), cached_max=cached_max,
                         new_max=new_max)
    ids_h, pos_h = metadata.prepare_prefill(seqs, bs, device="cpu")
    host = _snapshot()
    ids_d, pos_d = prepare_prefill_device(seqs, bs, device="cuda")
    torch.cuda.synchronize()
    dev = _snapshot()
    _same(host, dev)
    assert torch.equal(ids_h, ids_d.cpu()) and torch.equal(pos_h, pos_d.cpu())
    assert pos_d.dtype == torch.int64 and ids_d.dtype == torch.int64


def test_prefill_metadata_warmup_without_pages():
    say("prefill metadata warmup")
    rng = random.Random(5)
    seqs = _prefill_seqs(rng, 4, 256, pool=64, cached_max=0, new_max=300, with_tables=False)
    ids_h, pos_h = metadata.prepare_prefill(seqs, 256, device="cpu")
    host = _snapshot()
    ids_d, pos_d = prepare_prefill_device(seqs, 256, device="cuda")
    torch.cuda.synchronize()
    dev = _snapshot()
    _same(host, dev)
    assert dev["slot_mapping"].numel() == 0 and dev["block_tables"] is None
    assert torch.equal(pos_h, pos_d.cpu())


def _decode_seqs(rng, n, bs, pool):
    pages = list(range(pool))
    rng.shuffle(pages)
    nxt, seqs = 0, []
    for i in range(n):
        L = rng.choice([1, bs, bs + 1, 2 * bs, rng.randint(1, 9 * bs)])
        need = (L + bs - 1) // bs
        seqs.append(Sequence([rng.randint(0, 1000) for _ in range(L)],
                             block_table=pages[nxt:nxt + need]))
        nxt += need
    return seqs


@pytest.mark.parametrize("n,bs", [(1, 256), (13, 256), (512, 256), (40, 16)])
def test_decode_metadata_equals_host_builder(n, bs, monkeypatch):
    say(f"decode metadata n={n} bs={bs}")
    monkeypatch.setattr(Sequence, "block_size", bs)
    rng = random.Random(n + bs)
    seqs = _decode_seqs(rng, n, bs, pool=n * 10)
    ids_h, pos_h = metadata.prepare_decode(seqs, bs, device="cpu")
    host = _snapshot()
    ids_d, pos_d = prepare_decode_device(seqs, bs, device="cuda")
    torch.cuda.synchronize()
    dev = _snapshot()
    _same(host, dev)
    assert torch.equal(ids_h, ids_d.cpu()) and torch.equal(pos_h, pos_d.cpu())


class _Buffers:
    """The static buffers and bucket rule of a DecodeGraphRunner."""

    def __init__(self, max_bs, width, buckets):
        dev = "cuda"
        self.buckets = buckets
        self.positions = torch.full((max_bs,), 123, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.full((max_bs,), 77, dtype=torch.int32, device=dev)
        self.context_lens = torch.full((max_bs,), 55, dtype=torch.int32, device=dev)
        self.block_tables = torch.full((max_bs, width), 99, dtype=torch.int32, device=dev)

    def bucket(self, bs):
        return next(x for x in self.buckets if x >= bs)


def test_decode_metadata_into_graph_buffers_pads_like_run_model(monkeypatch):
    say("decode metadata into graph buffers")
    monkeypatch.setattr(Sequence, "block_size", 256)
    rng = random.Random(9)
    seqs = _decode_seqs(rng, 5, 256, pool=80)
    metadata.prepare_decode(seqs, 256, device="cpu")
    host = _snapshot()
    buf = _Buffers(32, 12, [1, 2, 4, 8, 16, 32])
    ids, pos = prepare_decode_device(seqs, 256, device="cuda", into=buf)
    torch.cuda.synchronize()
    dev = _snapshot()
    w = host["block_tables"].shape[1]
    assert torch.equal(dev["slot_mapping"], host["slot_mapping"])
    assert torch.equal(dev["context_lens"], host["context_lens"])
    assert torch.equal(dev["block_tables"][:, :w], host["block_tables"])
    assert dev["block_tables"][:, w:].eq(99).all()           # stale tail columns untouched
    sm, cl = buf.slot_mapping.cpu(), buf.context_lens.cpu()
    assert sm[5:8].eq(-1).all() and cl[5:8].eq(0).all()       # padded up to the bucket (8)
    assert sm[8:].eq(77).all() and cl[8:].eq(55).all()        # beyond the bucket: untouched
    assert buf.block_tables[5:].eq(99).all()                  # padded rows' tables untouched
    assert buf.positions[5:].eq(123).all()
    assert pos.cpu().tolist() == [len(s) - 1 for s in seqs]
