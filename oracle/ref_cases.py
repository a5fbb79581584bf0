"""Equations and shapes compiled against the reference CPU header (oracle/_ref).

The lists follow the reference's own test matrices so the oracle is pinned on
exactly the routes the reference exercises:

* ``EINSUM_CASES``     -- tests/test_einsum.py:22-129 (plus the batched
  partial-tile case it keeps skipped at :165-166, which the CPU header
  computes once the planner's guard is gone);
* ``ATTENTION_CASES``  -- tests/test_llm_ops.py:34-62;
* ``BROADCAST_CASES``  -- tests/test_llm_ops.py:115-125 (on the CPU route
  these are C=1 matmuls, builder.py:375-376);
* ``CHAIN_CASES``      -- the linear-attention steps of
  tests/test_llm_ops.py:81-107 at T=S in {96, 320};
* ``CONFIG_CASES``     -- the benchmark equations at reduced sizes, plus edge
  shapes (size-1 axes, scalar output, multi-axis contraction order);
* ``BENCH_SAMPLE``     -- the CPU baseline bench.py times: the whole of
  config 2 (``bji,bjk->bik``, b=16, j=777, i=1000, k=1536);
* ``BENCH_CONFIG_CASES`` -- every benchmark config at full size (config 2 is
  ``BENCH_SAMPLE``), which bench.py times on the reference CPU route beside
  each GPU row.  They are built but not run by the tests (config 3 alone is
  68.7 G multiply-adds).
"""

EINSUM_CASES = [
    ("ij,jk->ik", (32, 64), (64, 128)),
    ("ij,jk->ik", (256, 256), (256, 384)),
    ("i,j->ij", (64,), (96,)),
    ("i,i->", (256,), (256,)),
    ("ij,j->i", (32, 64), (64,)),
    ("i,ij->j", (32,), (32, 64)),
    ("ij,jk->ik", (16, 2048), (2048, 16)),
    ("ijk,jkl->il", (8, 16, 32), (16, 32, 64)),
    ("ji,jk->ik", (64, 32), (64, 128)),
    ("ij,kj->ik", (32, 64), (128, 64)),
    ("ji,kj->ik", (64, 32), (128, 64)),
    ("ji,jk->ik", (512, 500), (512, 64)),
    ("ij,jk->ki", (32, 64), (64, 48)),
    ("ai,ja->ij", (32, 16), (64, 32)),
    ("abc,cd->abd", (32, 16, 32), (32, 64)),
    ("bshd,bthd->bsht", (2, 128, 4, 64), (2, 128, 4, 64)),
    ("bshd,bthd->bsht", (2, 64, 4, 32), (2, 96, 4, 32)),
    ("bsht,bthd->bshd", (2, 128, 4, 128), (2, 128, 4, 64)),
    ("shd,thd->sht", (200, 1, 64), (128, 1, 64)),
    ("bij,bjk->bik", (32, 16, 32), (32, 32, 64)),
    ("bji,bjk->bik", (24, 32, 16), (24, 32, 64)),
    ("bij,bjk->bik", (64, 128, 128), (64, 128, 128)),
    ("bshd,bthd->bsht", (2, 128, 16, 64), (2, 128, 16, 64)),
    ("bihd,bjhd->bihj", (2, 128, 16, 128), (2, 128, 16, 128)),
    ("bihd,bjhd->bihj", (4, 128, 4, 128), (4, 128, 4, 128)),
    ("bnd,bmd->bnm", (8, 128, 64), (8, 128, 64)),
    ("bihd,bjhd->bihj", (2, 64, 4, 32), (2, 96, 4, 32)),
    ("bihj,bjhd->bihd", (2, 128, 16, 128), (2, 128, 16, 128)),
    ("bihj,bjhd->bihd", (4, 128, 4, 128), (4, 128, 4, 128)),
    ("bvhd,bhde->bvhe", (4, 128, 8, 64), (4, 8, 64, 64)),
    ("bnj,bjm->bnm", (8, 128, 128), (8, 128, 64)),
    ("bvhd,bvhe->bhde", (2, 128, 16, 128), (2, 128, 16, 128)),
    ("bvhd,bvhe->bhde", (4, 128, 4, 64), (4, 128, 4, 64)),
    ("vnd,vne->nde", (128, 8, 64), (128, 8, 64)),
    ("ij,jk->ik", (32, 20), (20, 128)),
    ("ai,ja->ij", (20, 16), (64, 20)),
    ("ji,jk->ik", (20, 32), (20, 128)),
    ("bij,bjk->bik", (8, 16, 20), (8, 20, 64)),
    ("i,i->i", (1000,), (1000,)),
    ("ts,ts->ts", (64, 48), (64, 48)),
    ("bshd,bshd->bshd", (2, 16, 8, 64), (2, 16, 8, 64)),
    ("ij,jk->ik", (250, 128), (128, 256)),
    ("ij,jk->ik", (256, 128), (128, 250)),
    ("ij,jk->ik", (250, 128), (128, 250)),
    ("ij,jk->ik", (200, 64), (64, 128)),
    ("ij,jk->ik", (128, 64), (64, 200)),
    ("ij,jk->ik", (200, 64), (64, 200)),
    ("ij,jk->ik", (1000, 64), (64, 128)),
    ("ij,jk->ik", (200, 20), (20, 200)),
    # reference-skipped batched partial tiles (test_einsum.py:165-166)
    ("bij,bjk->bik", (4, 200, 64), (4, 64, 128)),
]

ATTENTION_CASES = [
    ("bshd,bthd->bsht", (4, 16, 8, 64), (4, 16, 8, 64)),
    ("bsht,bthd->bshd", (4, 16, 8, 16), (4, 16, 8, 64)),
    ("bshd,hdk->bshk", (4, 16, 8, 64), (8, 64, 64)),
    ("bhs,bht->bst", (1, 20, 16), (1, 20, 24)),
    ("bhs,bht->bst", (4, 20, 16), (4, 20, 24)),
    ("bhsc,bcht->bsht", (2, 8, 16, 20), (2, 20, 8, 24)),
    ("bhsc,bhtc->bhst", (2, 8, 16, 20), (2, 8, 24, 20)),
    ("bhs,bht->bst", (2, 128, 256), (2, 128, 64)),
    ("bhs,bht->bst", (2, 130, 256), (2, 130, 64)),
    ("bhsc,bhtc->bhst", (2, 4, 16, 130), (2, 4, 256, 130)),
]

BROADCAST_CASES = [
    ("bsd,d->bsd", (2, 8, 64), (64,)),
    ("bsd,sd->bsd", (2, 8, 64), (8, 64)),
    ("bshd,sd->bshd", (2, 8, 4, 16), (8, 16)),
    ("hqk,h->hqk", (8, 16, 16), (8,)),
    ("bsd,d->bsd", (2, 16, 512), (512,)),
    ("bshd,sd->bshd", (4, 32, 8, 64), (32, 64)),
]

CHAIN_CASES = [
    ("tn,sn->ts", (96, 64), (96, 64)),
    ("ts,ts->ts", (96, 96), (96, 96)),
    ("ts,sp->tp", (96, 96), (96, 128)),
    ("tn,sn->ts", (320, 64), (320, 64)),
    ("ts,ts->ts", (320, 320), (320, 320)),
    ("ts,sp->tp", (320, 320), (320, 128)),
]

CONFIG_CASES = [
    # benchmark equations at reduced sizes
    ("bji,bjk->bik", (2, 77, 100), (2, 77, 153)),
    ("bshd,bthd->bsht", (2, 48, 4, 32), (2, 40, 4, 32)),
    ("ts,ts->ts", (128, 96), (128, 96)),
    ("bsd,d->bsd", (2, 32, 96), (96,)),
    ("bshd,sd->bshd", (2, 16, 4, 32), (16, 32)),
    ("tn,sn->ts", (160, 32), (144, 32)),
    ("ts,sp->tp", (160, 144), (144, 48)),
    # edge shapes
    ("ij,jk->ik", (1, 1), (1, 1)),
    ("ij,jk->ik", (1, 7), (7, 1)),
    ("i,i->", (1,), (1,)),
    ("i,i->", (1000,), (1000,)),
    ("bi,bi->b", (33, 65), (33, 65)),
    ("bij,bkj->bki", (3, 17, 9), (3, 5, 9)),
    ("ikj,jlk->il", (5, 6, 7), (7, 8, 6)),
    ("ab,ba->ab", (9, 13), (13, 9)),
    ("ai,bj->abij", (3, 5), (4, 6)),
    ("bi,bj->bij", (4, 7), (4, 9)),
    ("abc,cd->adb", (5, 6, 7), (7, 8)),
    ("ij,jk->ki", (129, 33), (33, 65)),
    ("xyz,zyw->wx", (3, 4, 5), (5, 4, 6)),
]

BENCH_SAMPLE = ("bji,bjk->bik", (16, 777, 1000), (16, 777, 1536))

BENCH_CONFIG_CASES = [
    ("ij,jk->ik", (256, 256), (256, 256)),                          # 1
    BENCH_SAMPLE,                                                   # 2
    ("bshd,bthd->bsht", (4, 2048, 32, 128), (4, 2048, 32, 128)),    # 3
    ("ts,ts->ts", (8192, 8192), (8192, 8192)),                      # 4a
    ("bsd,d->bsd", (8, 4096, 4096), (4096,)),                       # 4b
    ("tn,sn->ts", (4096, 128), (4096, 128)),                        # 5.1
    ("ts,ts->ts", (4096, 4096), (4096, 4096)),                      # 5.2
    ("ts,sp->tp", (4096, 4096), (4096, 128)),                       # 5.3
    ("bshd,sd->bshd", (2, 4096, 32, 128), (4096, 128)),             # 5.R
]

REF_CASES = (EINSUM_CASES + ATTENTION_CASES + BROADCAST_CASES + CHAIN_CASES
             + CONFIG_CASES + [BENCH_SAMPLE])
