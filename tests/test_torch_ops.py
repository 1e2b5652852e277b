"""The torch custom-op binding (libjacq_kivi_torch.so) on the CPU: schemas,
the fail-closed rejection table (through the ``_check`` twins, which run every
check except GPU residency and the device architecture), the GPU-only
dispatch of the real ops, and the residual-slot allocator
(source_patch.py:3047-3098)."""
from __future__ import annotations

import random

import pytest

torch = pytest.importorskip("torch")

from jacq_amd import torch_ops  # noqa: E402


@pytest.fixture(scope="module")
def ops():
    return torch_ops.load()


# The reference's registrations (source_patch.py:2797-2870): argument names in order.
DECODE = ["Q", "BLOCK_TABLE", "K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES", "V_CODE_PAGES",
          "V_SCALE_PAGES", "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH", "V_RESIDUAL_SCRATCH", "SEQ_LEN",
          "O"]
POOL = ["K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES", "V_CODE_PAGES", "V_SCALE_PAGES",
        "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH", "V_RESIDUAL_SCRATCH"]
SCHEMAS = {
    "kivi_decode_dsl": DECODE,
    "kivi_decode_sparse_retained_dsl": ["Q", "RETAINED_BLOCK_TABLE"] + POOL
    + ["SEQ_LEN", "NUM_RETAINED_PAGES", "O"],
    "kivi_decode_batched_dsl": ["Q", "SEQ_LENS", "BLOCK_TABLE"] + POOL + ["NUM_QUERIES", "O"],
    "kivi_cache_write_dsl": POOL + ["NEW_K", "NEW_V", "SLOT_MAPPING", "BLOCK_TABLE", "SEQ_LEN"],
    "kivi_cache_write_jac_dsl": POOL + ["NEW_K", "NEW_V", "SLOT_MAPPING", "BLOCK_TABLE",
                                        "SEQ_LEN"],
    "kivi_cache_write_batched_dsl": POOL + ["NEW_K", "NEW_V", "SLOT_MAPPING", "BLOCK_TABLE",
                                            "START_SEQ_LEN", "NUM_NEW"],
    "kivi_cache_write_batched_jac_dsl": POOL + ["NEW_K", "NEW_V", "SLOT_MAPPING", "BLOCK_TABLE",
                                                "START_SEQ_LEN", "NUM_NEW"],
}


@pytest.mark.parametrize("name", list(SCHEMAS))
def test_schema_matches_the_reference_registration(ops, name):
    for op_name in (name, name + "_check"):
        schema = getattr(ops, op_name).default._schema
        args = schema.arguments
        assert [a.name for a in args] == SCHEMAS[name], op_name
        writes = {a.name for a in args if a.alias_info is not None and a.alias_info.is_write}
        expect = {"O"} if "decode" in name else set(POOL)
        assert writes == expect, op_name
        assert len(schema.returns) == 0


# ---- valid CPU argument sets (v1 lane: page 32, group 32, R 128, 124-entry table) ----

def _pool(nkv=8, pages=6):
    h = torch.float16
    return dict(kc=torch.zeros(pages, nkv, 32, 64, dtype=torch.uint8),
                ks=torch.zeros(pages, nkv, 128, dtype=h), kz=torch.zeros(pages, nkv, 128, dtype=h),
                vc=torch.zeros(pages, nkv, 32, 64, dtype=torch.uint8),
                vs=torch.zeros(pages, nkv, 32, 4, dtype=h), vz=torch.zeros(pages, nkv, 32, 4, dtype=h),
                kscr=torch.zeros(nkv, 160, 128, dtype=h), vscr=torch.zeros(nkv, 160, 128, dtype=h))


PK = ("kc", "ks", "kz", "vc", "vs", "vz", "kscr", "vscr")


def _decode_args(nh=40, nkv=8):
    return dict(q=torch.zeros(nh, 128, dtype=torch.float16), bt=torch.zeros(124, dtype=torch.int32),
                **_pool(nkv), seq_len=1000, out=torch.zeros(nh, 128))


def _call(ops, name, a):
    op = getattr(ops, name + "_check")
    if name == "kivi_decode_dsl":
        return op(a["q"], a["bt"], *[a[k] for k in PK], a["seq_len"], a["out"])
    if name == "kivi_decode_sparse_retained_dsl":
        return op(a["q"], a["rbt"], *[a[k] for k in PK], a["seq_len"], a["retained"], a["out"])
    if name == "kivi_decode_batched_dsl":
        return op(a["q"], a["seq_lens"], a["bt"], *[a[k] for k in PK], a["nq"], a["out"])
    if name in ("kivi_cache_write_dsl", "kivi_cache_write_jac_dsl"):
        return op(*[a[k] for k in PK], a["nk"], a["nv"], a["slots"], a["bt"], a["seq_len"])
    return op(*[a[k] for k in PK], a["nk"], a["nv"], a["slots"], a["bt"], a["start"], a["n"])


def _args(name, nh=40, nkv=8):
    if name == "kivi_decode_dsl":
        return _decode_args(nh, nkv)
    if name == "kivi_decode_sparse_retained_dsl":
        a = _decode_args(nh, nkv)
        a.update(rbt=a.pop("bt"), retained=4)
        return a
    if name == "kivi_decode_batched_dsl":
        nq = 5
        return dict(q=torch.zeros(nq, nh, 128, dtype=torch.float16),
                    seq_lens=torch.arange(996, 1001, dtype=torch.int32),
                    bt=torch.zeros(124, dtype=torch.int32), **_pool(nkv), nq=nq,
                    out=torch.zeros(nq, nh, 128))
    if name in ("kivi_cache_write_dsl", "kivi_cache_write_jac_dsl"):
        return dict(**_pool(nkv), nk=torch.zeros(nkv, 128, dtype=torch.float16),
                    nv=torch.zeros(nkv, 128, dtype=torch.float16),
                    slots=torch.zeros(1, dtype=torch.int64), bt=torch.zeros(124, dtype=torch.int32),
                    seq_len=300)
    n = 40
    return dict(**_pool(nkv), nk=torch.zeros(n, nkv, 128, dtype=torch.float16),
                nv=torch.zeros(n, nkv, 128, dtype=torch.float16),
                slots=torch.zeros(n, dtype=torch.int64), bt=torch.zeros(124, dtype=torch.int32),
                start=500, n=n)


@pytest.mark.parametrize("name", list(SCHEMAS))
def test_valid_arguments_pass_every_check(ops, name):
    _call(ops, name, _args(name))
    if "jac" not in name:  # the TP=2 local-rank geometry (20 q / 4 kv heads)
        _call(ops, name, _args(name, 20, 4))


def _t(shape, dtype=torch.float16):
    return torch.zeros(*shape, dtype=dtype)


# (op, changes to the valid arguments, text the error must hold)
REJECT = [
    # dtypes
    ("kivi_decode_dsl", dict(q=_t((40, 128), torch.float32)), "Q must be fp16"),
    ("kivi_decode_dsl", dict(bt=_t((124,), torch.int64)), "BLOCK_TABLE must be int32"),
    ("kivi_decode_dsl", dict(kc=_t((6, 8, 32, 64), torch.int8)), "K_CODE_PAGES must be uint8"),
    ("kivi_decode_dsl", dict(vz=_t((6, 8, 32, 4), torch.float32)), "V_ZERO_PAGES must be fp16"),
    ("kivi_decode_dsl", dict(kscr=_t((8, 160, 128), torch.float32)),
     "K_RESIDUAL_SCRATCH must be fp16"),
    ("kivi_decode_dsl", dict(out=_t((40, 128))), "O must be fp32"),
    # geometry and shapes
    ("kivi_decode_dsl", dict(q=_t((32, 128)), out=_t((32, 128), torch.float32)),
     "supports global NH/NKV 40/8 or TP=2 local-rank NH/NKV 20/4; got NH=32 NKV=8"),
    ("kivi_decode_dsl", dict(q=_t((20, 128)), out=_t((20, 128), torch.float32)),
     "got NH=20 NKV=8"),
    ("kivi_decode_dsl", dict(q=_t((40, 64))), "Q dim 1 must be 128"),
    ("kivi_decode_dsl", dict(kc=_t((0, 8, 32, 64), torch.uint8)),
     "K_CODE_PAGES dim 0 (page storage capacity) must be positive"),
    ("kivi_decode_dsl", dict(kc=_t((8,), torch.uint8)), "K_CODE_PAGES must expose NKV at dim 1"),
    ("kivi_decode_dsl", dict(ks=_t((6, 8, 64))), "K_SCALE_PAGES dim 2 must be 128"),
    ("kivi_decode_dsl", dict(kz=_t((5, 8, 128))), "K_ZERO_PAGES dim 0 must be 6"),
    ("kivi_decode_dsl", dict(vc=_t((6, 8, 16, 64), torch.uint8)), "V_CODE_PAGES dim 2 must be 32"),
    ("kivi_decode_dsl", dict(vs=_t((6, 8, 32, 8))), "V_SCALE_PAGES dim 3 must be 4"),
    ("kivi_decode_dsl", dict(vscr=_t((8, 128, 128))), "V_RESIDUAL_SCRATCH dim 1 must be 160"),
    ("kivi_decode_dsl", dict(out=_t((40, 128, 1), torch.float32)), "O rank mismatch"),
    ("kivi_decode_dsl", dict(q=_t((128, 40)).t()), "Q must be contiguous for jac_launch"),
    # block table and length (source_patch.py:692-707)
    ("kivi_decode_dsl", dict(bt=_t((2, 62), torch.int32)), "BLOCK_TABLE rank mismatch"),
    ("kivi_decode_dsl", dict(seq_len=0), "SEQ_LEN must be in [1, 4096]"),
    ("kivi_decode_dsl", dict(seq_len=4097), "SEQ_LEN must be in [1, 4096]"),
    ("kivi_decode_dsl", dict(seq_len=4096, bt=_t((123,), torch.int32)),
     "BLOCK_TABLE dim 0 must be at least 124"),
    ("kivi_decode_dsl", dict(seq_len=160, bt=_t((0,), torch.int32)),
     "BLOCK_TABLE dim 0 must be at least 1"),
    # sparse-retained
    ("kivi_decode_sparse_retained_dsl", dict(rbt=_t((100,), torch.int32)),
     "RETAINED_BLOCK_TABLE dim 0 must be 124"),
    ("kivi_decode_sparse_retained_dsl", dict(rbt=_t((124,), torch.int64)),
     "RETAINED_BLOCK_TABLE must be int32"),
    ("kivi_decode_sparse_retained_dsl", dict(retained=125),
     "NUM_RETAINED_PAGES must be in [0, OLD_BLOCKS]"),
    ("kivi_decode_sparse_retained_dsl", dict(retained=-1),
     "NUM_RETAINED_PAGES must be in [0, OLD_BLOCKS]"),
    ("kivi_decode_sparse_retained_dsl", dict(retained=7),
     "NUM_RETAINED_PAGES cannot exceed physical page storage capacity"),
    ("kivi_decode_sparse_retained_dsl", dict(seq_len=5000),
     "SEQ_LEN must be in [1, 4096] for the KIVI sparse-retained DSL ABI"),
    # batched decode (one sequence, up to 160 causal queries)
    ("kivi_decode_batched_dsl", dict(q=_t((5, 40, 128), torch.float32)), "Q must be fp16"),
    ("kivi_decode_batched_dsl", dict(seq_lens=_t((5,), torch.int64)), "SEQ_LENS must be int32"),
    ("kivi_decode_batched_dsl", dict(q=_t((40, 128))),
     "Q rank mismatch for the batched KIVI DSL decode ABI"),
    ("kivi_decode_batched_dsl", dict(nq=0), "NUM_QUERIES must be in [1, MAX_QUERIES]"),
    ("kivi_decode_batched_dsl", dict(nq=161), "NUM_QUERIES must be in [1, MAX_QUERIES]"),
    ("kivi_decode_batched_dsl", dict(nq=4), "Q dim 0 must be 4"),
    ("kivi_decode_batched_dsl", dict(seq_lens=torch.tensor([9, 9, 9, 0, 9], dtype=torch.int32)),
     "SEQ_LENS[3] must be in [1, 4096] for the batched KIVI DSL decode ABI, got 0"),
    ("kivi_decode_batched_dsl", dict(seq_lens=torch.tensor([9, 9, 9, 9, 4100],
                                                            dtype=torch.int32)),
     "SEQ_LENS[4] must be in [1, 4096]"),
    ("kivi_decode_batched_dsl", dict(bt=_t((20,), torch.int32)),
     "BLOCK_TABLE dim 0 must be at least 27"),
    # single-token writer
    ("kivi_cache_write_dsl", dict(slots=_t((1,), torch.int32)), "SLOT_MAPPING must be int64"),
    ("kivi_cache_write_dsl", dict(nk=_t((8, 128), torch.float32)), "NEW_K must be fp16"),
    ("kivi_cache_write_dsl", dict(slots=_t((2,), torch.int64)),
     "SLOT_MAPPING must contain exactly one decode token"),
    ("kivi_cache_write_dsl", dict(nk=_t((4, 128))), "NEW_K dim 0 must be 8"),
    ("kivi_cache_write_dsl", dict(nv=_t((8, 64))), "NEW_V dim 1 must be 128"),
    ("kivi_cache_write_dsl", dict(seq_len=0), "SEQ_LEN must be in [1, 4096]"),
    ("kivi_cache_write_dsl", dict(seq_len=4096, bt=_t((100,), torch.int32)),
     "BLOCK_TABLE dim 0 must be at least 124"),
    ("kivi_cache_write_dsl", dict(**{k: v for k, v in _pool(nkv=6).items()},
                                  nk=_t((6, 128)), nv=_t((6, 128))),
     "supports global NH/NKV 40/8 or TP=2 local-rank NH/NKV 20/4; got NH=20 NKV=6"),
    ("kivi_cache_write_jac_dsl", dict(**{k: v for k, v in _pool(nkv=4).items()},
                                      nk=_t((4, 128)), nv=_t((4, 128))),
     "K_CODE_PAGES dim 1 must be 8"),
    # batched writer
    ("kivi_cache_write_batched_dsl", dict(n=0), "NUM_NEW must be in [1, RESIDUAL_SCRATCH]"),
    ("kivi_cache_write_batched_dsl", dict(n=161), "NUM_NEW must be in [1, RESIDUAL_SCRATCH]"),
    ("kivi_cache_write_batched_dsl", dict(nk=_t((39, 8, 128))), "NEW_K dim 0 must be 40"),
    ("kivi_cache_write_batched_dsl", dict(slots=_t((39,), torch.int64)),
     "SLOT_MAPPING must contain exactly NUM_NEW entries for the batched KIVI DSL writer"),
    ("kivi_cache_write_batched_jac_dsl", dict(slots=_t((39,), torch.int64)),
     "SLOT_MAPPING must contain exactly NUM_NEW entries for kivi_cache_write_batched_jac_dsl"),
    ("kivi_cache_write_batched_dsl", dict(start=-1),
     "START_SEQ_LEN + NUM_NEW must be in [0, 4096] for the batched KIVI DSL writer lane"),
    ("kivi_cache_write_batched_jac_dsl", dict(start=-1),
     "START_SEQ_LEN + NUM_NEW must be in [0, 4096] for kivi_cache_write_batched_jac_dsl"),
    ("kivi_cache_write_batched_dsl", dict(start=4060),
     "SEQ_LEN must be in [1, 4096] for KIVI BLOCK_TABLE validation"),
    ("kivi_cache_write_batched_dsl", dict(start=3000, bt=_t((50,), torch.int32)),
     "BLOCK_TABLE dim 0 must be at least 91"),
]


@pytest.mark.parametrize("name,change,text", REJECT,
                         ids=[f"{i}-{r[0][5:]}" for i, r in enumerate(REJECT)])
def test_rejection_table(ops, name, change, text):
    a = _args(name)
    a.update(change)
    with pytest.raises(RuntimeError) as e:
        _call(ops, name, a)
    assert text in str(e.value), str(e.value)


def test_real_ops_do_not_run_on_cpu_tensors(ops):
    """The ops are registered for the GPU backend only: CPU tensors find no
    kernel, so nothing runs and nothing falls back."""
    a = _decode_args()
    with pytest.raises(NotImplementedError, match="CPU"):
        ops.kivi_decode_dsl(a["q"], a["bt"], *[a[k] for k in PK], 1000, a["out"])
    w = _args("kivi_cache_write_dsl")
    with pytest.raises(NotImplementedError, match="CPU"):
        ops.kivi_cache_write_dsl(*[w[k] for k in PK], w["nk"], w["nv"], w["slots"], w["bt"], 300)


# ---- residual-slot allocator ----

def test_slots_are_stable_per_request():
    s = torch_ops.residual_slots(4)
    assert s.assign(["a", "b", "c"], [], None) == [0, 1, 2]
    assert s.assign(["c", "a", "b"], [], None) == [2, 0, 1]
    assert s.slot_of("b") == 1 and s.slot_of("zz") == -1
    assert (s.num_mapped(), s.num_free()) == (3, 0)


def test_finished_slots_return_last_freed_first():
    s = torch_ops.residual_slots(4)
    s.assign(["a", "b", "c"], [], None)
    # b then c finish: free list [1, 2]; d takes 2, e takes 1, f the next new index
    assert s.assign(["a", "d", "e", "f"], ["b", "c", "never-seen"], None) == [0, 2, 1, 3]
    assert s.num_free() == 0


def test_requests_missing_from_the_active_set_are_reclaimed_in_first_mapped_order():
    s = torch_ops.residual_slots(3)
    s.assign(["a", "b", "c"], [], None)
    # a and b are no longer active: freed in that order, so x (popped last) gets 1
    assert s.assign(["c", "x"], [], ["c", "x"]) == [2, 1]
    assert s.slot_of("a") == -1 and s.slot_of("b") == -1 and s.num_free() == 1


def test_pressure_reclaim_frees_requests_absent_from_the_step():
    s = torch_ops.residual_slots(2)
    s.assign(["a", "b"], [], None)
    # full, and nothing finished: a and b are not in this step, so they go
    assert s.assign(["c", "d"], [], None) == [1, 0]
    assert s.slot_of("a") == -1 and s.slot_of("b") == -1


def test_exhaustion_raises_not_implemented():
    s = torch_ops.residual_slots(2)
    with pytest.raises(NotImplementedError, match=r"ran out of residual slots \(max_seqs=2\)"):
        s.assign(["a", "b", "c"], [], None)
    with pytest.raises(RuntimeError, match="max_seqs >= 1"):
        torch_ops.residual_slots(0)


def test_random_serving_trace_keeps_slots_unique_and_stable():
    """A random admission / finish trace within max_num_seqs: no two live
    requests share a slot, every slot is below max_seqs, and a request keeps
    its slot for its whole life."""
    rng = random.Random(7)
    max_seqs = 8
    s = torch_ops.residual_slots(max_seqs)
    live: dict[str, int] = {}
    nxt = 0
    for step in range(400):
        finished = [r for r in live if rng.random() < 0.15]
        for r in finished:
            live.pop(r)
        while len(live) < max_seqs and rng.random() < 0.6:
            live[f"r{nxt}"] = -1
            nxt += 1
        step_ids = [r for r in live if rng.random() < 0.9] or list(live)[:1]
        active = list(live) if step % 3 == 0 else None
        got = s.assign(step_ids, finished, active)
        assert len(set(got)) == len(got) and all(0 <= x < max_seqs for x in got)
        for r, x in zip(step_ids, got):
            assert live[r] in (-1, x), (step, r)
            live[r] = x
        held = [v for v in live.values() if v >= 0]
        assert len(set(held)) == len(held), step


@pytest.mark.parametrize("name,change,text", REJECT[::3],
                         ids=[f"{i}-{r[0][5:]}" for i, r in enumerate(REJECT[::3])])
def test_python_mirrors_use_the_same_table(name, change, text):
    """jacq_amd.kivi's op mirrors validate through the ops' ``_check`` twins
    (kivi._validated), so they refuse what the ops refuse, with the same text,
    as KiviCheckError."""
    from jacq_amd import kivi

    class Mirror:
        def __getattr__(self, attr):
            return lambda *args: kivi._validated(attr[:-len("_check")], [], *args)

    a = _args(name)
    a.update(change)
    with pytest.raises(kivi.KiviCheckError) as e:
        _call(Mirror(), name, a)
    assert text in str(e.value), str(e.value)
