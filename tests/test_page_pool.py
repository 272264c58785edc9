"""Host logic of the paged packed cache: PagePool lifecycle, fences, ownership, and the
operator's metadata contract, all on the CPU.

Mirrors the pool semantics of ``turboquant_kv/page_pool.py:30-175`` and the
ownership tests of ``test_packed_model.py:278-343``:

* pages are allocated all-or-nothing under a per-request cap, refused rather
  than evicted (``PoolExhausted``);
* release bumps the page generation at once, so stale refs fail ``validate``
  (``StalePage``) even after the request id is reused;
* a released page returns to the free list only after the fence recorded behind
  its last reader completes ("awaiting fences");
* planted mutants of the pool (reclaim that ignores fences, release without the
  generation bump), made here on the CPU, are each caught.

``check_contract`` (``packed_attention.py:114-163``) runs on CPU tensors too:
every malformed handle is rejected with ``UnsupportedLayout`` before any launch.
"""
from __future__ import annotations

import threading
from types import SimpleNamespace

import pytest
import torch

from winnow_amd import packed_attention as pa
from winnow_amd import packed_backend as pb
from winnow_amd.page_pool import PagePool, PoolExhausted, StalePage


class Pending:
    """A fence that completes only when fired (a kernel still reading the page)."""

    def __init__(self):
        self.fired = False

    def query(self):
        return self.fired

    def synchronize(self):
        self.fired = True


def pool(pages=2, fence=None, cap=None, S=4):
    return PagePool(num_layers=1, num_pages=pages, num_kv_heads=1, page_size=S, nb_k=4, nb_v=4,
                    device="cpu", fence_factory=fence, max_pages_per_request=cap)


def test_layout_matches_the_reference_pool():
    p = PagePool(num_layers=3, num_pages=10, num_kv_heads=8, page_size=16, nb_k=64, nb_v=96, device="cpu")
    assert p.k_pages.shape == (3, 10, 8, 16, 64) and p.k_pages.dtype == torch.uint8
    assert p.v_pages.shape == (3, 10, 8, 16, 96)
    assert p.k_norms.shape == (3, 10, 8, 16) and p.k_norms.dtype == torch.float16
    assert p.bytes() == 3 * 10 * 8 * 16 * (64 + 96 + 2 + 2)
    assert p.bytes_per_token() == 3 * 8 * (64 + 96 + 2 + 2)
    d = PagePool(num_layers=1, num_pages=4, num_kv_heads=2, page_size=8, nb_k=32, nb_v=32, device="cpu",
                 dense_dtype=torch.bfloat16)
    assert d.dense and d.k_norms is None and d.k_pages.dtype == torch.bfloat16


def test_make_pool_sizes_from_a_model_config():
    cfg = SimpleNamespace(num_hidden_layers=2, num_key_value_heads=4, num_attention_heads=16, hidden_size=2048,
                          head_dim=128)
    p = pb.make_pool(cfg, bit_width=4, num_pages=5, page_size=16, device="cpu")
    assert p.k_pages.shape == (2, 5, 4, 16, 64)
    p6 = pb.make_pool(cfg, bit_width=6, num_pages=5, page_size=16, device="cpu")
    assert p6.v_pages.shape[-1] == 96
    dense = pb.make_pool(cfg, bit_width=None, num_pages=5, page_size=16, device="cpu",
                         dense_dtype=torch.float16)
    assert dense.k_pages.shape[-1] == 128


def test_ensure_is_all_or_nothing_and_capped():
    p = pool(pages=3, cap=2)
    assert len(p.ensure("a", 5)) == 2              # 5 tokens at S=4: 2 pages
    with pytest.raises(PoolExhausted, match="cap"):
        p.ensure("a", 9)                          # 3 pages > cap 2
    assert p.stats()["owned"] == 2
    with pytest.raises(PoolExhausted):
        p.ensure("b", 8)                          # 2 pages, 1 free: nothing taken
    assert p.stats() == {"free": 1, "pending": 0, "owned": 2, "requests": 2, "total": 3}
    assert len(p.ensure("b", 4)) == 1


def test_released_page_waits_for_its_fence():
    ev = Pending()
    p = pool()
    p.ensure("a", 8)
    p.release("a", ev)
    with pytest.raises(PoolExhausted, match="awaiting fences"):
        p.ensure("b", 4)
    ev.fired = True
    assert p.ensure("b", 4)


def test_mutant_reclaim_ignoring_fences_is_caught(monkeypatch):
    monkeypatch.setattr(PagePool, "_fence_done", lambda self, f: True)
    ev = Pending()
    p = pool()
    p.ensure("a", 8)
    p.release("a", ev)
    reused = p.ensure("b", 4)                     # only the mutant allows this
    assert reused and not ev.query()


def _reuse():
    p = pool(pages=1)
    old = p.ensure("a", 4)
    p.release("a")                                 # host pool: the default fence is already complete
    assert p.ensure("a", 4)[0].page == old[0].page
    return p, old


def test_stale_refs_fail_after_request_id_reuse():
    p, old = _reuse()
    with pytest.raises(StalePage):
        p.validate("a", old)
    p.validate("a", p.held("a"))


def test_mutant_release_without_generation_bump_is_caught(monkeypatch):
    def no_bump(self, pages):
        self._holder[pages] = -1
    monkeypatch.setattr(PagePool, "_revoke", no_bump)
    p = pool(pages=1)
    old = p.ensure("a", 4)
    p.release("a")
    p.ensure("b", 4)
    with pytest.raises(StalePage):                # another owner holds it now: still caught
        p.validate("a", old)
    p.release("b")
    p.ensure("a", 4)
    p.validate("a", old)                          # same owner again: only the generation could tell


def test_release_batches_pages_behind_one_fence():
    evs = [Pending(), Pending()]
    it = iter(evs)
    p = pool(pages=6, fence=lambda: next(it))
    p.ensure("a", 8)
    p.ensure("b", 12)
    assert [r.page for r in p.held("a")] == [0, 1] and [r.page for r in p.held("b")] == [2, 3, 4]
    assert p.release("a") == 2 and p.release("b") == 3
    assert p.stats() == {"free": 1, "pending": 5, "owned": 0, "requests": 0, "total": 6}
    evs[1].fired = True                           # b's fence completes first
    assert p.reclaim() == 3
    assert [r.page for r in p.ensure("c", 16)] == [2, 3, 4, 5]   # lowest free pages first
    evs[0].fired = True
    assert p.reclaim() == 2 and p.stats()["free"] == 2


def test_validate_rejects_foreign_and_out_of_range_refs():
    p = pool(pages=4)
    a = p.ensure("a", 4)
    p.ensure("b", 4)
    with pytest.raises(StalePage, match="current owner 'a'"):
        p.validate("b", a)
    with pytest.raises(StalePage, match="outside"):
        p.validate("a", [type(a[0])(7, 0)])


def test_concurrent_ensure_and_release_keep_the_page_count():
    p = pool(pages=64, S=4)
    errors = []

    def worker(i):
        try:
            for k in range(50):
                name = f"r{i}-{k}"
                try:
                    p.ensure(name, 4 * (1 + (k % 3)))
                except PoolExhausted:
                    continue
                p.validate(name, p.held(name))
                p.release(name)
        except Exception as e:  # noqa: BLE001
            errors.append(e)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    p.reclaim()
    st = p.stats()
    assert st["owned"] == 0 and st["free"] + st["pending"] == 64


# -- the operator's metadata contract on host tensors --------------------------

def host_kv(B=2, Hkv=2, D=64, S=16, lens=(20, 3), bw=4, P=4):
    nb = D * bw // 8
    table = torch.full((B, 2), -1, dtype=torch.int32)
    table[0] = torch.tensor([0, 1])
    table[1, 0] = 2
    q = pa.Quantizer(torch.eye(D), torch.zeros(2 ** bw), bw)
    kv = pa.PackedKV(torch.zeros(P, Hkv, S, nb, dtype=torch.uint8), torch.zeros(P, Hkv, S, dtype=torch.float16),
                     torch.zeros(P, Hkv, S, nb, dtype=torch.uint8), torch.zeros(P, Hkv, S, dtype=torch.float16),
                     table, torch.tensor(lens, dtype=torch.int32), q, q, D)
    return torch.zeros(B, 4, 1, D), kv


def _with(kv, **kw):
    return pa.PackedKV(**{**kv.__dict__, **kw})


def test_contract_accepts_a_well_formed_handle():
    q, kv = host_kv()
    pa.check_contract(q, kv)


@pytest.mark.parametrize("mutate", [
    lambda q, kv: (q[..., :32], kv),                                                  # head_dim mismatch
    lambda q, kv: (q[:, :3], kv),                                                     # Hq % Hkv
    lambda q, kv: (q[:, :, 0], kv),                                                   # q not 4-D
    lambda q, kv: (q, _with(kv, page_table=kv.page_table.long())),                    # int64 table
    lambda q, kv: (q, _with(kv, seq_lens=kv.seq_lens + 100)),                         # longer than the table
    lambda q, kv: (q, _with(kv, k_norms=kv.k_norms.float())),                         # fp32 norms
    lambda q, kv: (q, _with(kv, k_pages=kv.k_pages[..., :16])),                       # wrong NB
    lambda q, kv: (q, _with(kv, k_quant=pa.Quantizer(kv.k_quant.Pi, torch.zeros(8), 4))),   # 8 != 2**4 entries
    lambda q, kv: (q, _with(kv, k_quant=pa.Quantizer(kv.k_quant.Pi.double(), kv.k_quant.centroids, 4))),
    lambda q, kv: (q, _with(kv, page_table=torch.tensor([[0, 9], [2, -1]], dtype=torch.int32))),  # page id >= P
    lambda q, kv: (q, _with(kv, page_table=torch.tensor([[0, -1], [2, -1]], dtype=torch.int32))),  # used slot -1
])
def test_contract_rejects_before_launch(mutate):
    q, kv = host_kv()
    q, kv = mutate(q, kv)
    with pytest.raises(pa.UnsupportedLayout):
        pa.check_contract(q, kv)


def test_host_mirrors_are_what_the_range_checks_read():
    q, kv = host_kv()
    bad = _with(kv, page_table_host=torch.tensor([[0, 7], [2, -1]], dtype=torch.int32))
    with pytest.raises(pa.UnsupportedLayout):
        pa.check_contract(q, bad)
    pa.check_contract(q, bad, check_ranges=False)


def test_decode_dispatch_has_no_host_fallback():
    q, kv = host_kv()
    with pytest.raises(RuntimeError, match="HIP device"):
        pb.select_decode_backend(q, kv, "auto")
    with pytest.raises(ValueError):
        pb.select_decode_backend(q, kv, "no_such_backend")
    with pytest.raises(pa.UnsupportedLayout):
        pa.packed_decode_attention(q, kv, 1.0)      # host tensors never reach a kernel
    dense = pa.DenseKV(torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16), torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16),
                       torch.zeros(1, 2, dtype=torch.int32), torch.tensor([20], dtype=torch.int32), 128)
    qd = torch.zeros(1, 4, 1, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        pb.select_decode_backend(qd, dense, "auto")
    with pytest.raises(ValueError):
        pb.select_decode_backend(qd, dense, "hip_packed")


def test_unsupported_models_are_rejected():
    ok = SimpleNamespace(architectures=["Qwen2ForCausalLM"], hidden_size=1024, num_attention_heads=8, head_dim=128)
    pb.check_model(ok, 4)
    with pytest.raises(pb.UnsupportedModel):
        pb.check_model(SimpleNamespace(**{**ok.__dict__, "architectures": ["LlamaForCausalLM"]}), 4)
    with pytest.raises(pb.UnsupportedModel):
        pb.check_model(SimpleNamespace(**{**ok.__dict__, "use_sliding_window": True}), 4)
    with pytest.raises(ValueError):                 # 15 * 3 bits is not a whole number of bytes
        pb.check_model(SimpleNamespace(**{**ok.__dict__, "head_dim": 15}), 3)


def test_paged_cache_builds_its_table_from_the_pool_and_refuses_stale_owners():
    p = PagePool(num_layers=1, num_pages=8, num_kv_heads=1, page_size=4, nb_k=4, nb_v=4, device="cpu")
    p.ensure("a", 6)
    p.ensure("b", 3)
    cache = pb.PagedPackedCache(p, ["a", "b"], [5, 2], k_quant=None, v_quant=None, head_dim=8)
    meta = cache.begin(1, torch.device("cpu"))
    assert meta.table_host.shape == (2, 2) and meta.table_host.dtype == torch.int32
    assert meta.table_host[0].tolist() == [r.page for r in p.held("a")]
    assert meta.table_host[1, 0] == p.held("b")[0].page and meta.table_host[1, 1] == -1
    assert meta.seq_host.tolist() == [6, 3] and meta.start_host.tolist() == [5, 2]
    assert torch.equal(meta.table, meta.table_host) and torch.equal(meta.seq, meta.seq_host)
    short = pb.PagedPackedCache(p, ["b"], [4], k_quant=None, v_quant=None, head_dim=8)
    with pytest.raises(StalePage):                  # 5 tokens need 2 pages, b holds 1
        short.begin(1, torch.device("cpu"))
    p.release("b")
    gone = pb.PagedPackedCache(p, ["b"], [0], k_quant=None, v_quant=None, head_dim=8)
    with pytest.raises(StalePage):                  # released: holds nothing
        gone.begin(1, torch.device("cpu"))


def test_append_range_check_reads_host_metadata():
    """Positions past the table row or pages outside the pool are refused before launch
    (the reference raises in its gather, packed_backend.py:144)."""
    table = torch.tensor([[3, 1, -1], [0, -1, -1]], dtype=torch.int32)
    pb._positions_in_range(torch.tensor([30, 10]), table, 2, 4, 16)         # b0: 30,31 on page 1
    pb._positions_in_range(torch.tensor([0, 0]), table, 0, 4, 16)           # nothing appended
    with pytest.raises(pa.UnsupportedLayout, match="sequence 1"):
        pb._positions_in_range(torch.tensor([0, 15]), table, 2, 4, 16)      # b1: 16 needs column 1 (-1)
    with pytest.raises(pa.UnsupportedLayout, match="outside its 3-page"):
        pb._positions_in_range(torch.tensor([47, 0]), table, 2, 4, 16)      # 48 is past 3 pages
    with pytest.raises(pa.UnsupportedLayout, match="outside"):
        pb._positions_in_range(torch.tensor([0, 0]), table, 1, 3, 16)       # page 3 of a 3-page pool
    with pytest.raises(pa.UnsupportedLayout):
        pb._positions_in_range(torch.tensor([-1, 0]), table, 1, 4, 16)


def test_page_range_check_reads_only_live_slots():
    """Slots past cdiv(len, S) may hold anything (-1 padding, stale ids); a live slot
    outside [0, P) or a length beyond the table is an error."""
    table = torch.tensor([[3, 1, -1, 99], [0, -1, -1, -1]], dtype=torch.int32)
    pa.check_page_ranges(torch.tensor([17, 16], dtype=torch.int32), table, 4, 16)
    pa.check_page_ranges(torch.tensor([0, 0], dtype=torch.int32), table, 4, 16)
    with pytest.raises(pa.UnsupportedLayout, match="sequence 0"):
        pa.check_page_ranges(torch.tensor([33, 16], dtype=torch.int32), table, 4, 16)
    with pytest.raises(pa.UnsupportedLayout, match="sequence 1"):
        pa.check_page_ranges(torch.tensor([17, 17], dtype=torch.int32), table, 4, 16)
    with pytest.raises(pa.UnsupportedLayout, match="sequence 0"):
        pa.check_page_ranges(torch.tensor([17, 16], dtype=torch.int32), table, 3, 16)
    with pytest.raises(pa.UnsupportedLayout, match="out of range"):
        pa.check_page_ranges(torch.tensor([65, 0], dtype=torch.int32), table, 4, 16)
    with pytest.raises(pa.UnsupportedLayout, match="out of range"):
        pa.check_page_ranges(torch.tensor([-1, 0], dtype=torch.int32), table, 4, 16)
