"""KV-store scatter on the GPU: bit-exact parity with the oracle
(k_cache.view(-1, D)[slot] = key, slot -1 skipped; attention.py:10-40)."""
import numpy as np
import pytest
import torch

from gpu_utils import GOLDEN, bits, from_bits, oracle_store, say
from nanovllm_amd import _lib, store_kvcache
from nanovllm_amd.workloads import kv_store_case

pytestmark = pytest.mark.gpu


def _run_and_check(case, what):
    c = case.to("cuda")
    key0, value0 = bits(c.key).copy(), bits(c.value).copy()
    ek, ev = oracle_store(case.key, case.value, case.k_cache, case.v_cache, case.slot_mapping)
    say(what)
    store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(c.k_cache), ek, err_msg=f"{what}: k_cache")
    np.testing.assert_array_equal(bits(c.v_cache), ev, err_msg=f"{what}: v_cache")
    np.testing.assert_array_equal(bits(c.key), key0)
    np.testing.assert_array_equal(bits(c.value), value0)


def test_store_qwen3_layer_4096_tokens():
    case = kv_store_case()            # 4096 tokens, 64 pages, 205 slots = -1
    assert int((case.slot_mapping == -1).sum()) == 205
    _run_and_check(case, "kv_store 4096 tok, 5% skip")


@pytest.mark.parametrize("n_tokens", [1, 1279, 2001, 2560, 5121, 9000])
def test_store_every_tokens_per_thread_grid(n_tokens):
    # 2 KiB rows: 1 token per thread up to 1280 tokens, then 2, 4 and 8 (the
    # grid stays within 640 workgroups), including partial last workgroups
    pages = (n_tokens + 1000 + 255) // 256
    case = kv_store_case(seed=12, n_tokens=n_tokens, num_blocks=pages, skip=n_tokens // 20)
    _run_and_check(case, f"kv_store {n_tokens} tok")


def test_store_value_is_packed_qkv_view():
    # v is a view of the packed qkv: row stride (16 + 2*8) * 128 = 4096 elements
    case = kv_store_case(seed=11, n_tokens=777, value_row_stride=4096)
    assert case.value.stride(0) == 4096 and case.value.stride(1) == 128
    _run_and_check(case, "kv_store strided value")


def test_store_guide_matrix_fixture():
    data = np.load(f"{GOLDEN}/store_small.npz")
    for ci in range(3):
        key = from_bits(data[f"c{ci}_key"])
        value = from_bits(data[f"c{ci}_value"])
        kc = from_bits(data[f"c{ci}_k_cache"])
        vc = from_bits(data[f"c{ci}_v_cache"])
        slots = torch.from_numpy(data[f"c{ci}_slots"]).cuda()
        say(f"kv_store guide matrix case {ci} shape {tuple(key.shape)}")
        store_kvcache(key, value, kc, vc, slots)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(kc), data[f"c{ci}_expect_k"])
        np.testing.assert_array_equal(bits(vc), data[f"c{ci}_expect_v"])


@pytest.mark.parametrize("hkv,hd", [(3, 128), (1, 8), (2, 72)])
def test_store_other_row_sizes(hkv, hd):
    # 768 B rows (48 chunks: generic kernel), 16 B rows, 288 B rows
    case = kv_store_case(seed=5, n_tokens=300, num_blocks=4, hkv=hkv, hd=hd, skip=30)
    _run_and_check(case, f"kv_store hkv={hkv} hd={hd}")


def test_store_float32_and_int64_slots():
    gen = torch.Generator().manual_seed(3)
    key = torch.randn(50, 2, 16, generator=gen)
    value = torch.randn(50, 2, 16, generator=gen)
    slots = torch.randperm(64, generator=gen)[:50]
    slots[::7] = -1
    kc = torch.zeros(4, 16, 2, 16)
    vc = torch.zeros(4, 16, 2, 16)
    ek, ev = kc.clone().view(-1, 32), vc.clone().view(-1, 32)
    valid = slots >= 0
    ek[slots[valid]] = key.view(50, 32)[valid]
    ev[slots[valid]] = value.view(50, 32)[valid]
    kg, vg = kc.cuda(), vc.cuda()
    say("kv_store f32 int64 slots")
    store_kvcache(key.cuda(), value.cuda(), kg, vg, slots.cuda())  # int64 slot tensor
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(-1, 32), ek) and torch.equal(vg.cpu().view(-1, 32), ev)


def test_store_duplicate_and_out_of_range_slots_do_not_fault():
    # graph capture stores with an all-zero slot_mapping (model_runner.py:230,240-243):
    # duplicates are a race.  Each thread copies one 16-byte chunk (the Triton
    # reference races per element), so every chunk of the row comes from one of
    # the competing tokens.  Slots past the cache and negative values other
    # than -1 are skipped.
    gen = torch.Generator().manual_seed(9)
    n = 64
    key = torch.randn(n, 8, 128, generator=gen).to(torch.bfloat16).cuda()
    value = torch.randn(n, 8, 128, generator=gen).to(torch.bfloat16).cuda()
    kc = torch.zeros(2, 256, 8, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    say("kv_store duplicate slots")
    store_kvcache(key, value, kc, vc, torch.zeros(n, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    chunks = kc.view(-1, 1024)[0].view(128, 8)
    cand = key.view(n, 128, 8)
    for c in range(128):
        assert (cand[:, c] == chunks[c]).all(dim=1).any(), f"chunk {c} from no token"
    vchunks = vc.view(-1, 1024)[0].view(128, 8)
    for c in range(128):
        assert (value.view(n, 128, 8)[:, c] == vchunks[c]).all(dim=1).any()
    assert kc.view(-1, 1024)[1:].eq(0).all()
    kc.zero_(); vc.zero_()
    slots = torch.tensor([512, 10**6, -5, 3] + [-1] * (n - 4), dtype=torch.int32, device="cuda")
    say("kv_store out-of-range slots")
    store_kvcache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    flat = kc.view(-1, 1024)
    assert torch.equal(flat[3], key[3].view(-1))
    assert flat.ne(0).any(dim=1).sum().item() == 1


def test_store_empty_batch_is_a_no_op():
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16, device="cuda")
    e = torch.empty(0, 8, 128, dtype=torch.bfloat16, device="cuda")
    store_kvcache(e, e, kc, kc.clone(), torch.empty(0, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert kc.eq(0).all()


def test_store_rejects_bad_layouts():
    kc = torch.zeros(2, 16, 2, 8, dtype=torch.bfloat16, device="cuda")
    key = torch.zeros(4, 2, 8, dtype=torch.bfloat16, device="cuda")
    slots = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(AssertionError):
        store_kvcache(key.transpose(1, 2).contiguous().transpose(1, 2), key, kc, kc.clone(), slots)
    with pytest.raises(AssertionError):
        store_kvcache(key, key, kc, kc.clone(), slots[:3])
    with pytest.raises(_lib.NvkError):
        store_kvcache(key.cpu(), key.cpu(), kc.cpu(), kc.cpu(), slots.cpu())
