"""Planner restatement: recipes for the benchmark equations derived by hand
from builder.py:185-604, the reference's codegen gate strings, its error
contracts, and agreement with the oracle's independently written recipe."""
import os

import pytest
import torch

import oracle
from pto_einsum import EinsumBuilder, planner
from ref_cases import REF_CASES


def recipe(eq, s0, s1, device="cuda"):
    r, swapped, _, _ = planner.plan_operand_order(eq, s0, s1, device)
    return r, swapped


def test_config1_plain_matmul():
    r, sw = recipe("ij,jk->ik", (256, 256), (256, 256))
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (1, 256, 256, 256)
    assert r["in_transpose_idxs"] == ((0, 1), (0, 1)) and r["out_transpose_idxs"] == (0, 1)
    assert r["in_nt"] == 2 and r["out_fusible"] == 0 and not sw


def test_config2_transposed_batched():
    r, sw = recipe("bji,bjk->bik", (16, 777, 1000), (16, 777, 1536))
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (16, 1000, 1536, 777)
    assert r["in_transpose_idxs"] == ((0, 2, 1), (0, 1, 2)) and r["out_transpose_idxs"] == (0, 1, 2)
    assert r["in_nt"] == 0 and r["out_fusible"] == 0 and not sw


def test_config2_has_no_batched_partial_tile_guard():
    # The reference raises "Partial tiles are ... single-batch" here
    # (builder.py:593-604); this build plans it.
    b = EinsumBuilder("bji,bjk->bik", [(16, 777, 1000), (16, 777, 1536)], torch.float32)
    b.parse_equation()
    assert b.recipe["I"] == 16


def test_config3_attention_scores():
    r, sw = recipe("bshd,bthd->bsht", (4, 2048, 32, 128), (4, 2048, 32, 128))
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (128, 2048, 2048, 128)
    assert r["in_transpose_idxs"] == ((0, 2, 1, 3), (0, 2, 3, 1))
    assert r["out_transpose_idxs"] == (0, 2, 1, 3)
    assert r["out_fusible"] == 1 and r["out_row_stride"] == 65536
    assert r["out_batch_sizes"] == (4, 32) and r["out_batch_strides"] == (134217728, 2048)
    assert r["in_nt"] == 1 and r["in0_row_stride"] == 4096 and r["in1_col_stride"] == 4096
    assert r["in0_batch_strides"] == (8388608, 128) and r["in1_batch_strides"] == (8388608, 128)


def test_config4a_hadamard():
    r, _ = recipe("ts,ts->ts", (8192, 8192), (8192, 8192))
    assert r["elementwise"] and r["n_elem"] == 67108864


def test_config4b_broadcast_gpu_and_cpu_routes():
    r, _ = recipe("bsd,d->bsd", (8, 4096, 4096), (4096,))
    assert r["broadcast"] and r["bc_mode"] == 0
    assert (r["bc_Cc"], r["bc_Rr"], r["bc_Inner"], r["bc_Outer"], r["bc_sizeB"]) == (4096, 32768, 134217728, 1, 4096)
    c, _ = recipe("bsd,d->bsd", (8, 4096, 4096), (4096,), device="cpu")
    assert not c["broadcast"]
    assert (c["I"], c["L0"], c["L1"], c["C"]) == (4096, 32768, 1, 1)
    assert c["in_transpose_idxs"] == ((2, 0, 1), (0,)) and c["out_transpose_idxs"] == (1, 2, 0)


def test_config5_chain_and_rope():
    r, _ = recipe("tn,sn->ts", (4096, 128), (4096, 128))
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (1, 4096, 4096, 128)
    assert r["in_transpose_idxs"] == ((0, 1), (1, 0)) and r["in_nt"] == 1
    r, _ = recipe("ts,sp->tp", (4096, 4096), (4096, 128))
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (1, 4096, 128, 4096) and r["in_nt"] == 2
    r, _ = recipe("bshd,sd->bshd", (2, 4096, 32, 128), (4096, 128))
    assert r["broadcast"] and r["bc_mode"] == 0
    assert (r["bc_Cc"], r["bc_Rr"], r["bc_Inner"], r["bc_Outer"]) == (128, 32, 4096, 8192)
    assert r["bc_outer_dims"] == (2, 4096) and r["bc_outer_bstride"] == (0, 128)
    assert r["bc_sizeB"] == 524288
    c, _ = recipe("bshd,sd->bshd", (2, 4096, 32, 128), (4096, 128), device="cpu")
    assert (c["I"], c["L0"], c["L1"], c["C"]) == (524288, 64, 1, 1)


def test_broadcast_scalar_mode_and_no_caps():
    r, _ = recipe("hqk,h->hqk", (8, 16, 16), (8,))
    assert r["broadcast"] and r["bc_mode"] == 1 and r["bc_Inner"] == 256 and r["bc_Outer"] == 8
    # Cc = 8192 > 4096 and sizeB > 8192 stay on the broadcast route here.
    r, _ = recipe("bd,d->bd", (4, 8192), (8192,))
    assert r["broadcast"] and r["bc_Cc"] == 8192
    r, _ = recipe("hq,h->hq", (10000, 3), (10000,))
    assert r["broadcast"] and r["bc_mode"] == 1


@pytest.mark.parametrize("eq,s0,s1,field", [
    ("bihd,bjhd->bihj", (2, 128, 16, 128), (2, 128, 16, 128), "in_nt = 1"),   # test_einsum.py:291
    ("bihj,bjhd->bihd", (2, 128, 16, 128), (2, 128, 16, 128), "in_nt = 2"),   # :321
    ("bvhd,bvhe->bhde", (2, 128, 16, 128), (2, 128, 16, 128), "in_nt = 3"),   # :351
    ("bshd,bthd->bsht", (2, 128, 4, 64), (2, 128, 4, 64), "out_fusible = 1"),  # :370
    ("bihd,bjhd->bihj", (4, 128, 4, 128), (4, 128, 4, 128), "out_fusible = 1"),  # :371
    ("ij,jk->ik", (32, 64), (64, 128), "out_fusible = 0"),                      # :374
    ("ij,jk->ki", (32, 64), (64, 48), "out_fusible = 0"),                       # :375
])
def test_codegen_gate_strings(eq, s0, s1, field, tmp_path, monkeypatch):
    monkeypatch.setenv("EINSUM_BUILD_DIR", str(tmp_path))
    b = EinsumBuilder(eq, [s0, s1], torch.float32)
    b.parse_equation()
    b.generate_code()
    assert field in b.cpp_code


def test_disable_nt_switch(monkeypatch):
    monkeypatch.setenv("EINSUM_DISABLE_NT", "1")
    r, _ = recipe("bihd,bjhd->bihj", (2, 128, 16, 128), (2, 128, 16, 128))
    assert r["in_nt"] == 0


def test_operand_swap_and_disable(monkeypatch):
    # Output's innermost axis belongs to input0 -> swap exposes a fusible store.
    r, sw = recipe("bthd,bshd->bsht", (2, 64, 4, 32), (2, 48, 4, 32))
    assert sw and r["out_fusible"] == 1
    monkeypatch.setenv("EINSUM_DISABLE_OPERAND_SWAP", "1")
    r, sw = recipe("bthd,bshd->bsht", (2, 64, 4, 32), (2, 48, 4, 32))
    assert not sw


@pytest.mark.parametrize("eq,s0,s1,exc,msg", [
    ("ij,jk->k", (32, 64), (64, 128), ValueError, "single-operand reduction is not supported"),
    ("i...,i->i", (3,), (3,), ValueError, "subscripts should be in"),
    ("iij,jk->ik", (3, 3, 4), (4, 5), ValueError, "multiple times"),
    ("ij,jk->iz", (3, 4), (4, 5), ValueError, "not found in inputs"),
    ("ij,jk->ik", (3, 4, 1), (4, 5), ValueError, "Input0 requires 2 dimensions"),
    ("ij,jk->ik", (3, 4), (5, 5), ValueError, "mismatches for common subscript 'j'"),
])
def test_validation_contracts(eq, s0, s1, exc, msg):
    with pytest.raises(exc, match=msg):
        planner.parse_recipe(eq, s0, s1)


def test_dtype_contracts(tmp_path, monkeypatch):
    monkeypatch.setenv("EINSUM_BUILD_DIR", str(tmp_path))
    with pytest.raises(TypeError, match="Unsupported torch dtype"):
        b = EinsumBuilder("ij,jk->ik", [(2, 3), (3, 4)], torch.bfloat16)
        b.parse_equation()
        b.generate_code()
    with pytest.raises(TypeError, match="float16 is not supported on CPU"):
        b = EinsumBuilder("ij,jk->ik", [(2, 3), (3, 4)], torch.float16, device="cpu")
        b.parse_equation()
        b.generate_code()


def test_whitespace_equations_match_compact_form():
    a, _ = recipe("bshd, bthd -> bsht", (2, 8, 3, 4), (2, 8, 3, 4))
    b, _ = recipe("bshd,bthd->bsht", (2, 8, 3, 4), (2, 8, 3, 4))
    assert a == b


@pytest.mark.parametrize("eq,s0,s1", REF_CASES)
def test_cpu_recipe_agrees_with_oracle(eq, s0, s1):
    """The product planner's CPU-route recipe equals the oracle's own
    restatement: same perms, sizes and operand-swap decision."""
    r, sw = recipe(eq, s0, s1, device="cpu")
    o, osw = oracle.cpu_plan(eq, s0, s1)
    assert sw == osw
    if o["kind"] == "hadamard":
        assert r["elementwise"]
        return
    assert not r["elementwise"] and not r["broadcast"]
    assert tuple(r["in_transpose_idxs"][0]) == tuple(o["perm0"])
    assert tuple(r["in_transpose_idxs"][1]) == tuple(o["perm1"])
    assert tuple(r["out_transpose_idxs"]) == tuple(o["out_perm"])
    assert (r["I"], r["L0"], r["L1"], r["C"]) == (o["I"], o["L0"], o["L1"], o["C"])
    assert tuple(r["out_interpret_shape"]) == tuple(o["mid_shape"])
