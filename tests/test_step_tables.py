"""The step tables (glm53/tables.py step_rows / write_seed): the oracle against the
reference's own stated cases (tests/golden/step_rows_cases.json) and against what
the tables mean (CPU), then the HIP launch against the oracle (GPU)."""

import json
from pathlib import Path

import pytest
import torch

from oracle import reference as R

CASES = json.loads((Path(__file__).parent / "golden" / "step_rows_cases.json").read_text())


def _seed(case):
    seed = torch.full((case["S"], case["K"]), -1, dtype=torch.int32)
    for s, entries in enumerate(case["seed_entries"]):
        for j, v in entries:
            seed[s, j] = v
    return seed


@pytest.mark.parametrize("case", CASES["cases"], ids=[c["name"] for c in CASES["cases"]])
def test_oracle_step_rows_reference_cases(case):
    t = R.step_rows(case["slots"], case["positions"], case["S"], case["W"], case["K"], case["max_position"])
    assert t["positions"] == case["want_positions"]
    assert t["indptr"] == case["want_indptr"]
    assert t["slots"] == [s if s else -1 for s in case["slots"]]


def test_oracle_step_rows_reference_seed_case():
    case = CASES["seed_cases"][0]
    seed = _seed(case)
    t = R.step_rows(case["slots"], case["positions"], case["S"], case["W"], case["K"], case["max_position"],
                    seed=seed)
    assert t["indptr"] == case["want_indptr"] and t["topk"] == case["want_topk"]
    # the negative control of the reference's check: counts by position run past the
    # rows' valid entries
    bad = R.step_rows(case["slots"], case["positions"], case["S"], case["W"], case["K"], case["max_position"],
                      seed=seed, seed_by_position=True)
    assert bad["indptr"] == case["by_position_indptr"]
    rows = R.write_seed(t["topk"], t["indptr"], range(case["S"]), case["K"])
    for got, want in zip(rows, case["want_seed_rows"]):
        assert got[: len(want)] == want and all(v == -1 for v in got[len(want):])


def test_oracle_step_rows_pad_rows_and_ids():
    """Rows S..W-1 are pad rows; an in-step row with slot 0 keeps its position and id."""
    t = R.step_rows([9, 0], [3, 50], 2, 4, 2048, 40, ids_in=[7, 8])
    assert t["slots"] == [9, -1, -1, -1]
    assert t["positions"] == [3, 40, 0, 0]
    assert t["req_ids"] == [0, 1, 0, 0] and t["ids"] == [7, 8, -1, -1]
    assert t["ctx_len"] == [4, 0, 0, 0] and t["indptr"] == [0, 4, 4, 4, 4]


# ------------------------------------------------------------------------- GPU
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _gpu_tables(W, S, K, max_position, loc, pos, ids_in=None, seed=None, by_position=False):
    from sgl_amd_mono.k2.ops import StepRows

    st = StepRows(W, K, device=_dev())
    st(loc, pos, S, max_position, ids_in=ids_in, seed=seed, seed_by_position=by_position)
    torch.cuda.synchronize()
    return st


def _check_against_oracle(st, W, S, K, max_position, loc, pos, ids_in=None, seed=None, by_position=False):
    cpu = lambda t: None if t is None else t.cpu()  # noqa: E731
    want = R.step_rows(cpu(loc).tolist(), cpu(pos).tolist(), S, W, K, max_position,
                       ids_in=None if ids_in is None else cpu(ids_in).tolist(),
                       seed=cpu(seed), seed_by_position=by_position)
    assert st.slots.cpu().tolist() == want["slots"]
    assert st.positions.cpu().tolist() == want["positions"]
    assert st.req_ids.cpu().tolist() == want["req_ids"]
    assert st.indptr.cpu().tolist() == want["indptr"]
    assert st.ctx_len.cpu().tolist() == want["ctx_len"]
    if ids_in is not None:
        assert st.ids.cpu().tolist() == want["ids"]
    if seed is not None:
        n = want["indptr"][W]
        assert st.topk[:n].cpu().tolist() == want["topk"]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES["cases"], ids=[c["name"] for c in CASES["cases"]])
def test_gpu_step_rows_reference_cases(case):
    dev = _dev()
    loc = torch.tensor(case["slots"], dtype=torch.int64, device=dev)
    pos = torch.tensor(case["positions"], dtype=torch.int64, device=dev)
    st = _gpu_tables(case["W"], case["S"], case["K"], case["max_position"], loc, pos)
    assert st.positions.cpu().tolist() == case["want_positions"]
    assert st.indptr.cpu().tolist() == case["want_indptr"]


@pytest.mark.gpu
def test_gpu_step_rows_reference_seed_case():
    dev = _dev()
    case = CASES["seed_cases"][0]
    loc = torch.tensor(case["slots"], dtype=torch.int64, device=dev)
    pos = torch.tensor(case["positions"], dtype=torch.int64, device=dev)
    seed = _seed(case).to(dev)
    st = _gpu_tables(case["W"], case["S"], case["K"], case["max_position"], loc, pos, seed=seed)
    assert st.indptr.cpu().tolist() == case["want_indptr"]
    assert st.topk[:5].cpu().tolist() == case["want_topk"]
    bad = _gpu_tables(case["W"], case["S"], case["K"], case["max_position"], loc, pos, seed=seed, by_position=True)
    assert bad.indptr.cpu().tolist() == case["by_position_indptr"]
    out = torch.full((case["S"], case["K"]), 7, dtype=torch.int32, device=dev)
    st.write_seed(out, case["S"], torch.arange(case["S"], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    for got, want in zip(out.cpu().tolist(), case["want_seed_rows"]):
        assert got[: len(want)] == want and all(v == -1 for v in got[len(want):])


@pytest.mark.gpu
@pytest.mark.parametrize("W, S", [(2, 1), (4, 3), (4, 4), (8, 5), (32, 17), (32, 32)])
@pytest.mark.parametrize("with_seed", [False, True], ids=["positions", "seed"])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_gpu_step_rows_random_against_oracle(W, S, with_seed, ids_dtype):
    """Random steps as the reference's own table test draws them (a strided slot view, a
    padding slot, positions past max_position), with and without a reused top-k, and
    the by-position variant; then write_seed of every row."""
    dev = _dev()
    g = torch.Generator().manual_seed(W * 10 + S)
    K, max_position = 2048, 9000
    loc = torch.randint(1, 1 << 30, (3 * S,), generator=g)[::3]
    if S > 1:
        loc[S - 1] = 0
    pos = torch.randint(0, 12000, (S,), generator=g)
    pos[0] = 100
    ids_in = torch.randint(0, 150000, (S,), generator=g).to(ids_dtype)
    seed = None
    if with_seed:
        seed = torch.randint(0, 1 << 30, (S, K), generator=g, dtype=torch.int32)
        for s in range(S):
            seed[s, int(torch.randint(1, K + 1, (1,), generator=g)):] = -1
            seed[s, torch.randint(0, K, (40,), generator=g)] = -1  # holes inside
        seed = seed.to(dev)
    loc_d = torch.randint(1, 1 << 30, (3 * S,), generator=g).to(dev)
    loc_d[::3] = loc.to(dev)
    loc_v = loc_d[::3]  # a strided view, as SGLang's per-step draft slots
    pos, ids_in = pos.to(dev), ids_in.to(dev)
    st = _gpu_tables(W, S, K, max_position, loc_v, pos, ids_in=ids_in, seed=seed)
    _check_against_oracle(st, W, S, K, max_position, loc_v, pos, ids_in=ids_in, seed=seed)
    if with_seed:
        st2 = _gpu_tables(W, S, K, max_position, loc_v, pos, seed=seed, by_position=True)
        _check_against_oracle(st2, W, S, K, max_position, loc_v, pos, seed=seed, by_position=True)
        out = torch.full((W, K), 7, dtype=torch.int32, device=dev)
        rows_of = torch.arange(W, dtype=torch.int32, device=dev).flip(0)
        st.write_seed(out, W, rows_of)
        torch.cuda.synchronize()
        want = R.write_seed(st.topk.cpu().tolist(), st.indptr.cpu().tolist(), rows_of.cpu().tolist(), K)
        assert out.cpu().tolist() == want
