"""The C-ABI library (no GPU needed): it loads, exports every symbol include/bsgemm.h declares,
and rejects invalid arguments on the host before any HIP call."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

import bsa_mi355x as bsa
from bsa_mi355x import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bsgemm.h")
HEADERS = [HEADER, os.path.join(ROOT, "include", "bsgemm_timeline.h")]


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(bsg_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_and_library_exports_everything():
    lib = bsa.load()
    names = _declared()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_version():
    assert b"gfx950" in bsa.load().bsg_version()


def test_packed_bytes():
    lib = bsa.load()
    assert lib.bsg_packed_bytes(4096, 11008, 0) == 172 * 64 * 4096 * 2
    assert lib.bsg_packed_bytes(100, 1000, 0) == 16 * 64 * 112 * 2
    assert lib.bsg_packed_bytes(0, 64, 0) == -1
    assert lib.bsg_packed_bytes(16, 64, 7) == -1


def _resolve(bt, n, nblk, na, cu=256, plan=None):
    p = plan or _lib.Plan()
    rc = bsa.load().bsg_plan_resolve(bt, n, nblk, na, cu, ctypes.byref(p))
    return rc, p


def test_plan_resolve_auto_fills_every_field():
    rc, p = _resolve(16, 4096, 172, 86)
    assert rc == 0
    assert p.split_k >= 1 and p.cols_per_wave in (16, 32, 64, 128) and p.waves_per_group in (1, 2, 4, 8)
    assert p.depth in (1, 2, 4, 8) and p.rows_per_group == 16 and p.kind == 1
    assert _resolve(64, 4096, 64, 31)[1].rows_per_group == 64 and _resolve(64, 4096, 64, 31)[1].kind == 2
    assert _resolve(2, 4096, 64, 0)[1].split_k == 1
    # automatic plans use MFMA (kind 1) for small batches; kind 3 (dot products) when named,
    # with the batch rounded up to a power of two and enough waves to stage the list
    rc, p = _resolve(3, 4096, 64, 13)
    assert rc == 0 and (p.kind, p.rows_per_group) == (1, 16)
    rc, p = _resolve(3, 4096, 64, 13, plan=_lib.Plan(0, 0, 0, 0, 0, 3))
    assert rc == 0 and (p.kind, p.rows_per_group, p.split_k, p.waves_per_group) == (3, 4, 1, 4)
    rc, p = _resolve(2, 11008, 172, 172, plan=_lib.Plan(0, 0, 0, 0, 0, 3))
    assert rc == 0 and (p.kind, p.rows_per_group, p.waves_per_group) == (3, 2, 4)
    rc, p = _resolve(4, 11008, 172, 172, plan=_lib.Plan(0, 0, 0, 0, 0, 3))
    assert rc == 0 and (p.kind, p.rows_per_group, p.waves_per_group) == (3, 4, 8)


def test_plan_resolve_rejects():
    assert _resolve(0, 4096, 64, 1)[0] == _lib.BSG_ERR_ARG
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(0, 48, 0, 0, 0, 0))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(0, 0, 0, 0, 24, 0))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(0, 0, 0, 0, 0, 8))[0] == _lib.BSG_ERR_UNSUPPORTED
    # kind 7 (kind 6 with LDS activations): no split-K, and only tiles whose wave reduction fits
    # the waves' activation slots (at most 2 x depth subtiles) are compiled
    assert _resolve(64, 4096, 64, 1, plan=_lib.Plan(2, 48, 4, 2, 64, 7))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(64, 4096, 64, 1, plan=_lib.Plan(1, 96, 2, 2, 64, 7))[0] == _lib.BSG_ERR_UNSUPPORTED
    rc, p = _resolve(64, 4096, 64, 1, plan=_lib.Plan(0, 0, 0, 0, 0, 7))
    assert rc == 0 and p.as_tuple() == (1, 48, 4, 4, 64, 7)
    # kind 5 (variable-width column groups): no split-K, only its instantiated widths
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(2, 48, 4, 4, 16, 5))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(1, 80, 4, 4, 16, 5))[0] == _lib.BSG_ERR_UNSUPPORTED
    rc, p = _resolve(16, 4096, 64, 1, plan=_lib.Plan(0, 0, 0, 0, 0, 5))
    assert rc == 0 and p.as_tuple() == (1, 48, 4, 4, 16, 5)
    # kind 4 pairs the waves over channel halves: one wave has no partner
    assert _resolve(64, 4096, 64, 1, plan=_lib.Plan(0, 16, 1, 4, 64, 4))[0] == _lib.BSG_ERR_UNSUPPORTED
    # kind 3: no split-K, 1-8 rows, and its activation staging must hold the list
    assert _resolve(4, 4096, 64, 8, plan=_lib.Plan(2, 0, 0, 0, 0, 3))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(4, 4096, 64, 8, plan=_lib.Plan(0, 0, 0, 0, 16, 3))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(8, 4096, 2048, 2048, plan=_lib.Plan(0, 0, 0, 0, 0, 3))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert _resolve(16, 4096, 64, 1, plan=_lib.Plan(300, 0, 0, 0, 0, 0))[0] == _lib.BSG_ERR_UNSUPPORTED
    assert "plan" in _lib.last_error()


def _plan_doc_kinds():
    """kind -> its paragraph in the bsg_plan comment of include/bsgemm.h."""
    text = open(HEADER).read()
    doc = text[text.index("/* Launch plan of the GEMM."):text.index("typedef struct bsg_plan")]
    kinds = {}
    cur = None
    for line in doc.splitlines():
        m = re.match(r"\s*\*\s{5}(\d)\s{2}(.*)", line)
        if m:
            cur = int(m.group(1))
            kinds[cur] = m.group(2)
        elif cur is not None and re.match(r"\s*\*\s{8}\S", line):
            kinds[cur] += " " + line.split("*", 1)[1].strip()
        else:
            cur = None
    return kinds


def _accepted_kinds():
    """Every kind bsg_plan_resolve resolves with at least one tile, probing each kind's row
    counts with every other field left automatic."""
    out = set()
    for kind in range(0, 10):
        for bt, rows in ((16, 16), (64, 64), (32, 32), (4, 4)):
            if _resolve(bt, 4096, 64, 32, plan=_lib.Plan(0, 0, 0, 0, rows, kind))[0] == 0:
                out.add(kind)
                break
    return out


def test_header_documents_every_plan_kind():
    """Each kind the library accepts has its own paragraph in the header's bsg_plan comment, the
    header's split-K rule matches what the resolver enforces, and every kind the shipped plan
    table names is among them (a C caller reading the header can form any shipped plan)."""
    doc = _plan_doc_kinds()
    accepted = _accepted_kinds() - {0}
    assert accepted == {1, 2, 3, 4, 5, 6, 7}
    assert set(doc) == accepted, (sorted(doc), sorted(accepted))
    for kind in accepted:
        rows = 4 if kind == 3 else 16
        rc_sk2 = _resolve(rows, 4096, 64, 32, plan=_lib.Plan(2, 0, 0, 0, rows, kind))[0]
        single = "split_k must be 1" in doc[kind]
        assert (rc_sk2 == _lib.BSG_ERR_UNSUPPORTED) == single, (kind, rc_sk2, doc[kind])
    import json
    table = json.load(open(os.path.join(ROOT, "towards-batched-activation-sparsity_amd", "bsa_mi355x",
                                        "tuned_plans.json")))
    shipped = {e["plan"][5] for e in table["entries"]}
    assert shipped <= accepted and {5, 6} <= shipped
    # the kind-0 heuristic stated in the header
    assert _resolve(16, 4096, 64, 32)[1].kind == 1 and _resolve(64, 4096, 64, 32)[1].kind == 2


def test_workspace_bytes():
    lib = bsa.load()
    p = _lib.Plan(1, 32, 4, 4, 16, 1)
    assert lib.bsg_gemm_workspace_bytes(16, 4096, ctypes.byref(p)) == 0
    p = _lib.Plan(4, 32, 4, 4, 16, 1)
    tiles = 4096 // 32
    assert lib.bsg_gemm_workspace_bytes(16, 4096, ctypes.byref(p)) == 512 + tiles * 4 * 2 * 64 * 16
    p = _lib.Plan(2, 16, 8, 4, 64, 4)  # kind 4: 8 waves = 4 column groups x 2 channel halves
    assert lib.bsg_gemm_workspace_bytes(64, 4096, ctypes.byref(p)) == 256 + 64 * 2 * (4 * 4) * 64 * 16
    p = _lib.Plan(2, 16, 4, 4, 64, 2)  # kind 2: a work-group covers 16 * 4 columns
    tiles = 4096 // 64
    assert lib.bsg_gemm_workspace_bytes(64, 4096, ctypes.byref(p)) == 256 + tiles * 2 * (4 * 4) * 64 * 16
    assert lib.bsg_select_workspace_bytes(4096) == 1280  # 256 + 64 blocks x (score, energy)
    assert lib.bsg_select_workspace_bytes(0) == -1


FAKE = 1 << 40  # never dereferenced: every call below fails validation first


def test_gemm_rejects_bad_arguments_without_launching():
    lib = bsa.load()
    p = _lib.Plan(2, 32, 4, 4, 16, 1)
    ok = dict(x=FAKE, ldx=4096, bt=16, K=4096, wp=FAKE, N=4096, idx=FAKE, na=10, nad=None, y=FAKE, ldy=4096,
              dtype=0, ws=FAKE, ws_bytes=1 << 30)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.bsg_gemm(a["x"], a["ldx"], a["bt"], a["K"], a["wp"], a["N"], a["idx"], a["na"], a["nad"], a["y"],
                            a["ldy"], a["dtype"], a["ws"], a["ws_bytes"], ctypes.byref(p), None)

    assert call(dtype=3) == _lib.BSG_ERR_DTYPE
    assert call(x=None) == _lib.BSG_ERR_ARG
    assert call(K=100) == _lib.BSG_ERR_ALIGN
    assert call(ldx=4100) == _lib.BSG_ERR_ALIGN
    assert call(x=FAKE + 8) == _lib.BSG_ERR_ALIGN
    assert call(ldy=100) == _lib.BSG_ERR_ARG
    assert call(na=-1) == _lib.BSG_ERR_ARG
    assert call(na=5000) == _lib.BSG_ERR_ARG
    assert call(idx=None) == _lib.BSG_ERR_ARG
    assert call(ws=None) == _lib.BSG_ERR_WORKSPACE
    assert call(ws_bytes=16) == _lib.BSG_ERR_WORKSPACE
    assert call(K=200000) == _lib.BSG_ERR_UNSUPPORTED
    assert "workspace" in _lib.last_error() or "K" in _lib.last_error()

    def call_sorted(**kw):
        a = dict(ok, **kw)
        return lib.bsg_gemm_sorted(a["x"], a["ldx"], a["bt"], a["K"], a["wp"], a["N"], a["idx"], a["na"], a["nad"],
                                   a["y"], a["ldy"], a["dtype"], a["ws"], a["ws_bytes"], ctypes.byref(p), None)

    # the in-kernel sort takes at most BSG_MAX_NBLK / 2 entries
    assert call_sorted(na=_lib.MAX_NBLK // 2 + 1, K=64 * _lib.MAX_NBLK, ldx=64 * _lib.MAX_NBLK) == _lib.BSG_ERR_UNSUPPORTED
    assert "sort" in _lib.last_error()
    assert call_sorted(na=-1) == _lib.BSG_ERR_ARG
    assert call_sorted(idx=None) == _lib.BSG_ERR_ARG


def test_2d_entry_points_reject_bad_arguments_without_launching():
    lib = bsa.load()
    p = _lib.Plan(1, 16, 2, 4, 16, 1)
    ok = dict(x=FAKE, ldx=4096, bt=16, K=4096, wp=FAKE, N=4096, idx=FAKE, na=10, nad=None, nb=FAKE, nn=3, nnd=None,
              compact=0, y=FAKE, ldy=4096, dtype=0, ws=None, ws_bytes=0, plan=p)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.bsg_gemm_2d(a["x"], a["ldx"], a["bt"], a["K"], a["wp"], a["N"], a["idx"], a["na"], a["nad"],
                               a["nb"], a["nn"], a["nnd"], a["compact"], a["y"], a["ldy"], a["dtype"], a["ws"],
                               a["ws_bytes"], ctypes.byref(a["plan"]), None)

    assert call(nn=65) == _lib.BSG_ERR_ARG           # more blocks than ceil(N/64)
    assert call(nn=-1) == _lib.BSG_ERR_ARG
    assert call(nb=None) == _lib.BSG_ERR_ARG
    assert call(compact=1, ldy=100) == _lib.BSG_ERR_ARG  # compact Y needs nn * 64 columns
    assert call(ldy=100) == _lib.BSG_ERR_ARG             # in place needs N
    assert call(nn=0, nb=None) == _lib.BSG_OK            # no output block: nothing to launch
    wide = _lib.Plan(1, 32, 4, 4, 32, 2)                 # 128 columns per work-group
    assert call(plan=wide) == _lib.BSG_ERR_UNSUPPORTED
    assert "64" in _lib.last_error()
    assert lib.bsg_scatter_nblocks(FAKE, 100, 16, FAKE, 2, None, 4096, FAKE, 4096, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_scatter_nblocks(FAKE, 4096, 16, FAKE, 65, None, 4096, FAKE, 4096, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_scatter_nblocks(FAKE, 128, 16, FAKE, 2, None, 4096, FAKE, 100, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_scatter_nblocks(FAKE, 128, 16, FAKE, 0, None, 4096, FAKE, 4096, None) == _lib.BSG_OK
    assert lib.bsg_nmask_blocks(FAKE, 0, FAKE, FAKE, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_nmask_blocks(None, 64, FAKE, FAKE, None) == _lib.BSG_ERR_ARG


def test_bitmap_and_select_reject_bad_arguments():
    lib = bsa.load()
    p = _lib.Plan(1, 32, 4, 4, 16, 1)
    assert lib.bsg_gemm_bitmap(FAKE, 4096, 16, 4096, FAKE, 4096, None, 64, FAKE, 4096, 0, None, 0,
                               ctypes.byref(p), None) == _lib.BSG_ERR_ARG
    assert lib.bsg_gemm_bitmap(FAKE, 4096, 16, 4096, FAKE, 4096, FAKE, 65, FAKE, 4096, 0, None, 0,
                               ctypes.byref(p), None) == _lib.BSG_ERR_ARG
    assert lib.bsg_select_topk_l1(FAKE, 4096, 16, 4096, 8, FAKE, FAKE, 1, FAKE, 1024, None) == _lib.BSG_ERR_DTYPE
    assert lib.bsg_select_topk_l1(FAKE, 4096, 16, 4096, 8, FAKE, FAKE, 0, FAKE, 16, None) == _lib.BSG_ERR_WORKSPACE
    assert lib.bsg_select_topk_l1(FAKE, 4096, 16, 4096, -1, FAKE, FAKE, 0, FAKE, 1024, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_pack_weight(FAKE, 16, 64, 64, 1, 0, FAKE, 8, None) == _lib.BSG_ERR_ARG
    assert lib.bsg_workspace_init(None, 64, None) == _lib.BSG_ERR_ARG


def test_status_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.BSG_ERR_ARG)
    with pytest.raises(TypeError):
        _lib.check(_lib.BSG_ERR_DTYPE)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.BSG_ERR_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.BSG_ERR_HIP)
    _lib.check(0)


def test_kernel_tiles_and_config_shims():
    tiles = bsa.kernel_tiles()
    assert (1, 16, 32, 4, 4) in tiles and (1, 64, 64, 4, 2) in tiles and (2, 64, 16, 4, 4) in tiles
    from bsa_mi355x import runtime

    cfgs = runtime._PREPACK_AUTOTUNE_CONFIGS
    assert len(cfgs) == len(tiles)
    assert {"BLOCK_B", "BLOCK_N"} <= set(cfgs[0].kwargs) and cfgs[0].num_warps >= 1 and cfgs[0].num_stages >= 1


def test_make_plan_maps_reference_tiles():
    p = bsa.make_plan(4, 16, 64, 2, 3, bt=64)
    assert p.as_tuple() == (4, 64, 2, 4, 64, 0)   # BLOCK_B raised to cover the batch; stages -> depth 4
    assert bsa.make_plan().as_tuple() == (0, 0, 0, 0, 0, 0)
    assert bsa.n_keep_for_density(0.48, 64) == 31


def test_select_topk_rejects_bad_options():
    """Argument checks of bsg_select_topk run on the host (no device pointer is touched)."""
    lib = bsa.load()
    fake = 1 << 20  # never dereferenced: every case below fails its host checks first

    def call(opts, k=4, kdim=4096):
        rc = lib.bsg_select_topk(fake, kdim, 2, kdim, k, ctypes.byref(opts), fake, fake, 0, fake, 1 << 20, None)
        return rc, _lib.last_error()

    rc, msg = call(_lib.SelectOpts(7, 0.0, None, 1.0, 0.1, None, None))
    assert rc == _lib.BSG_ERR_UNSUPPORTED and "score" in msg
    rc, msg = call(_lib.SelectOpts(_lib.BSG_SCORE_L1, 0.5, None, 1.0, 0.1, None, None))
    assert rc == _lib.BSG_ERR_UNSUPPORTED
    rc, msg = call(_lib.SelectOpts(_lib.BSG_SCORE_ENERGY, 1.5, None, 1.0, 0.1, None, None))
    assert rc == _lib.BSG_ERR_ARG and "energy_keep" in msg
    rc, msg = call(_lib.SelectOpts(_lib.BSG_SCORE_L2_MEAN, 0.0, None, 1.0, 0.1, fake, None))
    assert rc == _lib.BSG_ERR_ARG and "channel_scale" in msg
    rc, msg = call(_lib.SelectOpts(_lib.BSG_SCORE_L2_MEAN, 0.0, None, 1.0, 0.1, None, None), kdim=32)
    assert rc == _lib.BSG_ERR_ARG
    rc, msg = call(_lib.SelectOpts(_lib.BSG_SCORE_L2_MEAN, 0.0, None, 1.0, 0.1, None, None), k=-1)
    assert rc == _lib.BSG_ERR_ARG


def test_shipped_library_has_no_timeline():
    """The shipped build exports the profiling hook but rejects it (its kernels carry no stamps)."""
    lib = bsa.load()
    assert lib.bsg_timeline_attach(None, 0, 0) == 0
    assert lib.bsg_timeline_attach(ctypes.c_void_p(0x1000), 1, 1) == _lib.BSG_ERR_UNSUPPORTED
