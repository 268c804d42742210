"""C-ABI boundary without a GPU: the library loads, exports what the headers
declare, classifies and plans dispatches, and rejects bad arguments on the
host before anything is launched."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT


def header_functions():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(iree_mi355x_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.library()
    declared = header_functions()
    assert declared == set(pkg.EXPORTED_SYMBOLS)
    for name in declared:
        assert getattr(lib, name) is not None


# Device-memory allocators, frees and fills of the HIP runtime: the C-ABI
# imports none of them (scratch comes from a caller workspace, or, for the
# allocation-free entry point, from a static device array).
ALLOCATING = ("hipMalloc", "hipMallocAsync", "hipMallocManaged",
              "hipMallocPitch", "hipExtMallocWithFlags", "hipHostMalloc",
              "hipMallocFromPoolAsync", "hipFree", "hipFreeAsync",
              "hipHostFree", "hipMemset", "hipMemsetAsync", "hipMemsetD32",
              "hipMemsetD32Async", "hipDeviceSynchronize")


def test_library_imports_no_allocator(pkg):
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", pkg.LIB_PATH],
                         check=True, capture_output=True, text=True).stdout
    imported = {line.split()[-1].split("@")[0] for line in out.splitlines()
                if line.strip()}
    assert "hipLaunchKernel" in imported  # the listing is the real one
    assert not imported & set(ALLOCATING), imported & set(ALLOCATING)


def test_missing_workspace_is_refused_before_launch(pkg):
    # split-K and GEMV plans need a workspace: none, or a short one, is
    # refused on the host (no device here: nothing could have launched)
    lib = pkg.library()
    for m, n, k in [(16, 4096, 4096), (1, 4096, 4096)]:
        need = lib.iree_mi355x_matmul_workspace_bytes(m, n, k, 0)
        assert need > 0
        st = lib.iree_mi355x_matmul_f16(FAKE, FAKE, FAKE, m, n, k, k, n, n, 0,
                                        None, 0, None)
        assert st == pkg.WORKSPACE_TOO_SMALL, pkg.last_error()
        assert str(need) in pkg.last_error() or "workspace" in pkg.last_error()
        # the query bounds every form; the f16 plan itself needs this much
        exact = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).workspace_bytes
        assert 0 < exact <= need
        st = lib.iree_mi355x_matmul_f16(FAKE, FAKE, FAKE, m, n, k, k, n, n, 0,
                                        FAKE, exact - 1, None)
        assert st == pkg.WORKSPACE_TOO_SMALL
        st = lib.iree_mi355x_w8a16_matmul(FAKE, FAKE, FAKE, FAKE, m, n, k, k,
                                          n, n, 0, None, 0, None)
        assert st == pkg.WORKSPACE_TOO_SMALL
    # an autotuner run of a split-K configuration likewise
    cfg = next(c for c in pkg.mfma_configs()
               if c.name == "f16_nn_64x128x64_w2x2_s4_sk")
    need = lib.iree_mi355x_matmul_mfma_config_workspace_bytes(
        cfg.index, 4, 64, 4096, 4096, 0)
    assert need > 0
    assert lib.iree_mi355x_matmul_mfma_config_split(
        cfg.index, 4, FAKE, FAKE, None, FAKE, 64, 4096, 4096, 4096, 4096,
        4096, 0, None, 0, None) == pkg.WORKSPACE_TOO_SMALL


def test_version_and_no_device_here(pkg):
    lib = pkg.library()
    assert b"gfx950" in lib.iree_mi355x_version()
    assert lib.iree_mi355x_device_count() >= 0


def test_executable_library_table(pkg):
    assert ctypes.sizeof(pkg.DispatchAttrs) == 24
    lib = pkg.executable_library()
    assert lib.header.contents.version == pkg.EXECUTABLE_LIBRARY_VERSION
    assert lib.imports.count == 0
    assert pkg.export_names() == ["matmul_f16", "matmul_i8", "w8a16_matmul",
                                  "attention_f16", "batch_matmul_f16"]
    for i in range(lib.exports.count):
        attrs = lib.exports.attrs[i]
        assert attrs.flags & 1  # RESOURCES_VALID
        assert 0 < attrs.lds_bytes <= 160 * 1024
        assert attrs.threads in (256, 512)
    # any other version: NULL, like the reference's exact-version rule
    assert pkg.executable_library(0x48580001) is None
    assert pkg.executable_library(pkg.EXECUTABLE_LIBRARY_VERSION + 1) is None


F16, I8, I32, F32 = 0, 1, 2, 3


@pytest.mark.parametrize("case,family,tile", [
    ((I8, I8, I32, 4096, 4096, 4096, 1), 1, (256, 256)),
    ((F16, F16, F16, 4096, 4096, 4096, 1), 1, (256, 256)),
    ((F16, F16, F32, 4096, 4096, 4096, 1), 1, (256, 256)),
    ((F16, F16, F16, 2048, 4096, 4096, 1), 1, (256, 128)),
    # C1: a measured entry (16 workgroups of 32x128, one split)
    ((F16, F16, F16, 128, 512, 256, 0), 1, (32, 128)),
    ((F16, F16, F16, 2048, 4096, 4096, 0), 1, (256, 128)),
    ((F16, F16, F16, 100, 512, 256, 0), 1, None),
    ((F16, F16, F16, 100, 500, 256, 0), 2, (64, 64)),
    ((F16, F16, F16, 17, 19, 23, 1), 2, (64, 64)),
    # GEMV: the half-wave form (32 lanes x 8 f16 per row) where it shrinks
    # the final sum, the full-wave form (64 lanes) otherwise
    ((F16, F16, F16, 1, 4096, 4096, 0), 3, (1, 256)),
    ((F16, F16, F16, 4, 11008, 4096, 0), 3, (4, 512)),
    ((F16, F16, F16, 5, 4096, 4096, 0), 1, None),
    ((F16, F16, F16, 5, 4090, 4096, 0), 2, (64, 64)),
    # int8 with row-major B: macro-tiles, and split-K tiles for skinny M
    ((I8, I8, I32, 4096, 4096, 4096, 0), 1, (256, 256)),
    ((I8, I8, I32, 1, 4096, 4096, 0), 1, None),
    ((I8, I8, I32, 16, 4096, 4096, 1), 1, None),
])
def test_planner_classification(pkg, case, family, tile):
    a, b, c, m, n, k, flags = case
    d = pkg.make_desc(a, b, c, m, n, k, flags)
    assert pkg.classify(d) == family
    p = pkg.plan(d)
    assert p.family == family
    if tile is None:  # ragged M: a split-K configuration (rows past M
        # masked), tile and split count by cost model
        assert p.config_name.decode().endswith("_sk") and p.splits >= 1
    else:
        assert (p.tile_m, p.tile_n) == tile
    name = p.config_name.decode()
    form = "tn" if flags & 1 else "nn"
    prefix = {1: ("i8_" if a == I8 else ("f16f32_" if c == F32 else "f16_")) + form + "_",
              2: "general_", 3: "gemv_"}[family]
    assert name.startswith(prefix), name
    if family == 1:
        # the chosen config really has this macro-tile and fits the LDS budget
        cfg = [x for x in pkg.mfma_configs() if x.name == name][0]
        assert (cfg.tile_m, cfg.tile_n) == (p.tile_m, p.tile_n)
        assert cfg.lds_bytes <= 160 * 1024


def test_planner_w8a16_and_unsupported_types(pkg):
    d = pkg.make_desc(F16, I8, F16, 1, 11008, 4096, 0, has_scale=True)
    p = pkg.plan(d)
    # half-wave form: 32 lanes x 16 int8 per row
    assert p.family == pkg.FAMILY_GEMV and p.tile_n == 512
    assert p.config_name == b"gemv_w8a16_r1_h2"
    assert p.workspace_bytes > 0 and p.splits > 1
    d = pkg.make_desc(F16, I8, F16, 512, 11008, 4096, 0, has_scale=True)
    p = pkg.plan(d)
    assert p.family == pkg.FAMILY_MFMA and p.config_name.startswith(b"w8a16_nn_")
    d = pkg.make_desc(F16, I8, F16, 512, 11008, 4096, pkg.B_TRANSPOSED,
                      has_scale=True)
    assert pkg.classify(d) == pkg.FAMILY_GENERAL
    for bad in ((F32, F32, F32), (I8, F16, F16), (F16, F16, I32), (I8, I8, F16)):
        d = pkg.make_desc(*bad, 64, 64, 64, 0)
        assert pkg.classify(d) == pkg.FAMILY_NONE
        with pytest.raises(pkg.MI355XError):
            pkg.plan(d)


def test_planner_lds_budget_and_alignment(pkg):
    # a budget below every macro-tile's LDS leaves the general kernel
    d = pkg.make_desc(I8, I8, I32, 4096, 4096, 4096, 1, lds_budget_bytes=32 * 1024)
    assert pkg.classify(d) == pkg.FAMILY_GENERAL
    d = pkg.make_desc(I8, I8, I32, 4096, 4096, 4096, 1, aligned=False)
    assert pkg.classify(d) == pkg.FAMILY_GENERAL
    d = pkg.make_desc(I8, I8, I32, 4096, 4096, 4096, 1, lds_budget_bytes=130 * 1024)
    p = pkg.plan(d)
    assert p.lds_bytes <= 130 * 1024 and p.family == pkg.FAMILY_MFMA


def test_planner_ranking_prefers_least_traffic(pkg):
    # 4096^3: every candidate has the same per-CU work; 256x256 moves least
    d = pkg.make_desc(I8, I8, I32, 4096, 4096, 4096, 1)
    p = pkg.plan(d)
    assert (p.tile_m, p.tile_n) == (256, 256)
    assert p.traffic_bytes == 4096 * 4096 * (16 + 16)
    assert p.workgroups == 256


@pytest.mark.parametrize("m,n,k,flags,want", [
    (2048, 4096, 4096, 0, b"f16_nn_256x128x64_w2x4_s2_m16"),
    (2048, 11008, 4096, 0,
     b"f16_nn_256x256x64_w2x4_s2_m16+256x128x64_w2x4_s2_m16"),
    (2048, 4096, 11008, 0, b"f16_nn_256x128x64_w2x4_s2_m16"),
    (4096, 4096, 4096, 0, b"f16_nn_256x256x64_w2x4_s2_m16"),
    (4096, 4096, 4096, 8, b"f16at_nn_256x256x64_w2x4_s2_m16"),
])
def test_planner_prefers_16x16_on_full_grids(pkg, m, n, k, flags, want):
    # Feed-bound f16 shapes whose tiles fill every CU: the 16x16 MFMA form
    # of the tile measured faster than the 32x32 one (same modeled time)
    p = pkg.plan(pkg.make_desc(F16, F16, F16, m, n, k, flags))
    assert p.config_name == want and p.splits == 1
    # a grid that leaves CUs idle keeps the 32x32 form
    p = pkg.plan(pkg.make_desc(F16, I8, F16, 512, 11008, 4096, 0,
                               has_scale=True))
    assert not p.config_name.endswith(b"_m16")


def column_split_parts(name):
    """Head and tail configuration names of a column split, named
    "<head>+<tail without the head's type and B form prefix>"."""
    head, tail = name.split("+")
    pre = head[:head.index("_", head.index("_") + 1) + 1]
    return head, pre + tail


def test_config_names_fit_the_plan(pkg):
    """Every configuration name, column splits included, fits the plan's
    63-character config_name, and each split's parts are listed."""
    names = [c.name for c in pkg.mfma_configs()]
    for name in names:
        assert len(name) <= 63, name
        if "+" in name:
            head, tail = column_split_parts(name)
            assert head in names and tail in names, name


COLUMN_SPLITS = [
    ((F16, F16, F16), 0, b"f16_nn_256x256x64_w2x4_s2_m16",
     b"f16_nn_256x128x64_w2x4_s2_m16", 8 * 22),
    ((F16, F16, F16), 1, b"f16_tn_256x256x64_w2x4_s2_m16",
     b"f16_tn_256x128x64_w2x4_s2_m16", 8 * 22),
    ((F16, F16, F16), 8, b"f16at_nn_256x256x64_w2x4_s2_m16",
     b"f16at_nn_256x128x64_w2x4_s2", 8 * 22),
    ((F16, F16, F16), 9, b"f16at_tn_256x256x64_w2x4_s2_m16",
     b"f16at_tn_256x128x64_w2x4_s2", 8 * 22),
    ((I8, I8, I32), 1, b"i8_tn_256x256x128_w2x4_s2_m16",
     b"i8_tn_256x128x128_w2x4_s2_m16", 8 * 22),
    ((I8, I8, I32), 0, b"i8_nn_256x256x128_w2x4_s2_m16",
     b"i8_nn_128x256x128_w2x4_s2", 16 * 11),
    ((F16, F16, F32), 0, b"f16f32_nn_256x256x64_w2x4_s2_m16",
     b"f16f32_nn_256x128x64_w2x4_s2_m16", 8 * 22),
    ((F16, F16, F32), 1, b"f16f32_tn_256x256x64_w2x4_s2_m16",
     b"f16f32_tn_256x128x64_w2x4_s2_m16", 8 * 22),
    ((F16, F16, F32), 8, b"f16f32at_nn_256x256x64_w2x4_s2_m16",
     b"f16f32at_nn_256x128x64_w2x4_s2", 8 * 22),
    ((F16, F16, F32), 9, b"f16f32at_tn_256x256x64_w2x4_s2_m16",
     b"f16f32at_tn_256x128x64_w2x4_s2", 8 * 22),
]


@pytest.mark.parametrize("types,flags,head,tail,tail_wgs", COLUMN_SPLITS)
def test_planner_column_split(pkg, types, flags, head, tail, tail_wgs):
    """C3 M=2048 N=11008: 344 tiles of 256x256 end in a round of 88; the
    plan runs the head over 8192 columns (one round of 256 tiles) and the
    tail tile over the last 2816 columns, with no workspace."""
    for k in (4096, 11008):
        p = pkg.plan(pkg.make_desc(*types, 2048, 11008, k, flags))
        pre = head[:head.index(b"_", head.index(b"_") + 1) + 1]
        assert p.config_name == head + b"+" + tail[len(pre):]
        assert p.workgroups == 256 + tail_wgs
        assert p.splits == 1 and p.workspace_bytes == 0
    # the head alone where its grid ends in whole rounds, or where the rest
    # needs more than one round of tail tiles (4096 x 11008: 352 tiles)
    for m, n in ((4096, 4096), (4096, 11008)):
        p = pkg.plan(pkg.make_desc(*types, m, n, 4096, flags))
        assert b"+" not in p.config_name, (m, n)
    # batched calls, and a chip of another CU count, take no column split
    # (W8A16 below: the model ranks the 128x256 tile first there, and the
    # split replaces it too)
    p = pkg.plan(pkg.make_desc(*types, 2048, 11008, 4096, flags, batch=2))
    assert b"+" not in p.config_name
    d = pkg.make_desc(*types, 2048, 11008, 4096, flags)
    d.num_cus = 128
    assert b"+" not in pkg.plan(d).config_name


def test_planner_column_split_w8a16(pkg):
    """W8A16 at 2048 x 11008: the model ranks 688 tiles of 128x256 first;
    the column split (one round of 256x256, one of 176 128x256 tiles)
    replaces it."""
    for k in (4096, 11008):
        p = pkg.plan(pkg.make_desc(F16, I8, F16, 2048, 11008, k, 0,
                                   has_scale=True))
        assert p.config_name == (b"w8a16_nn_256x256x64_w2x4_s3+"
                                 b"128x256x64_w2x4_s4")
        assert p.workgroups == 256 + 176 and p.workspace_bytes == 0
    # C5 M=512 has no whole round of 256x256 tiles: no split
    p = pkg.plan(pkg.make_desc(F16, I8, F16, 512, 11008, 4096, 0,
                               has_scale=True))
    assert b"+" not in p.config_name


def test_column_split_head_rule_on_the_cpu(pkg):
    """The composite runs only where its launcher can split: the named
    configuration with a shape it cannot split is refused before launch."""
    cfgs = {c.name: c for c in pkg.mfma_configs()}
    name = "f16_nn_256x256x64_w2x4_s2_m16+256x128x64_w2x4_s2_m16"
    idx = cfgs[name].index
    lib = pkg.library()
    # 4096^3: whole rounds of 256x256 tiles, nothing left for the tail
    assert lib.iree_mi355x_matmul_mfma_config_workspace_bytes(
        idx, 0, 4096, 4096, 4096, 0) == 0
    assert lib.iree_mi355x_matmul_mfma_config_split(
        idx, 0, 256, 256, None, 256, 4096, 4096, 4096, 4096, 4096, 4096, 0,
        None, 0, None) == pkg.UNSUPPORTED


def test_planner_rowdot_gemv(pkg):
    """Weights [N, K] (B_TRANSPOSED) with M <= 4: the row-dot GEMV, no
    workspace, where whole 16-byte segments tile K and x fits the LDS it is
    staged in (M x K x 2 <= 60 KiB); otherwise the MFMA or general path."""
    for (a, b, c), kw, tag in (((F16, F16, F16), {}, b"f16"),
                               ((F16, F16, F32), {}, b"f16f32"),
                               ((F16, I8, F16), {"has_scale": True},
                                b"w8a16")):
        for m, n, k in ((1, 11008, 4096), (4, 11008, 4096), (2, 4096, 11008),
                        (1, 1000, 1040)):
            p = pkg.plan(pkg.make_desc(a, b, c, m, n, k, pkg.B_TRANSPOSED,
                                       **kw))
            assert p.family == pkg.FAMILY_GEMV
            assert p.config_name == b"gemv_rowdot_" + tag + b"_r%d" % m
            assert p.workspace_bytes == 0 and p.splits == 1
            assert p.workgroups == min((n + 7) // 8, 512)
        # x 66 KB past the LDS it uses (W8A16 splits it over launches of 2
        # rows), K not a multiple of 16, too many rows
        for m, n, k in ((3, 4096, 11008 if tag != b"w8a16" else 40960),
                        (1, 1000, 1000),
                        (5 if tag != b"w8a16" else 17, 4096, 4096)):
            p = pkg.plan(pkg.make_desc(a, b, c, m, n, k, pkg.B_TRANSPOSED,
                                       **kw))
            assert b"rowdot" not in p.config_name, (m, n, k)
    # W8A16 up to 16 rows: launches of at most 8 rows each, as many as x's
    # LDS limit allows (7 at K = 4096), dealt evenly
    p = pkg.plan(pkg.make_desc(F16, I8, F16, 3, 4096, 11008,
                               pkg.B_TRANSPOSED, has_scale=True))
    assert p.config_name == b"gemv_rowdot_w8a16_r3"
    assert p.workgroups == 512 * 2 and p.lds_bytes == 2 * 11008 * 2
    for m, rows in ((5, 5), (7, 7), (8, 4), (12, 6), (16, 6)):
        p = pkg.plan(pkg.make_desc(F16, I8, F16, m, 11008, 4096,
                                   pkg.B_TRANSPOSED, has_scale=True))
        assert p.config_name == b"gemv_rowdot_w8a16_r%d" % m
        assert p.workgroups == 512 * ((m + rows - 1) // rows)
        assert p.lds_bytes == rows * 4096 * 2
    # x rows must be 16-byte aligned to be staged
    d = pkg.make_desc(F16, F16, F16, 1, 4096, 4096, pkg.B_TRANSPOSED)
    d.a_aligned16 = 0
    assert b"rowdot" not in pkg.plan(d).config_name


def test_mfma_config_table(pkg):
    cfgs = pkg.mfma_configs()
    assert len(cfgs) >= 8
    for c in cfgs:
        assert c.lds_bytes <= 160 * 1024
        assert c.tile_m % 32 == 0 and c.tile_n % 32 == 0
        assert c.threads in (256, 512)


def test_workspace_query(pkg):
    lib = pkg.library()
    # GEMV (M <= 4, B [K,N]) and split-K shapes use one; full tiles do not
    assert lib.iree_mi355x_matmul_workspace_bytes(1, 4096, 4096, 0) > 0
    assert lib.iree_mi355x_matmul_workspace_bytes(16, 4096, 4096, 0) > 0
    assert lib.iree_mi355x_matmul_workspace_bytes(2048, 4096, 4096, 0) == 0
    assert lib.iree_mi355x_matmul_workspace_bytes(4096, 4096, 4096, 1) == 0


def test_planner_split_k_for_skinny_shapes(pkg):
    # M = 16 cannot fill 256 CUs with output tiles: K is split and the
    # plan carries the split count and a workspace for the partials
    p = pkg.plan(pkg.make_desc(F16, F16, F16, 16, 4096, 4096, 0))
    assert p.family == pkg.FAMILY_MFMA and p.splits > 1
    assert p.config_name.endswith(b"_sk")
    assert p.splits * p.k_split >= 4096 and p.k_split % p.tile_k == 0
    assert p.workgroups >= 128 and p.workspace_bytes >= p.splits * 16 * 4096 * 4
    # large M: enough tiles, no split
    p = pkg.plan(pkg.make_desc(F16, F16, F16, 2048, 4096, 4096, 0))
    assert p.splits == 1 and p.workspace_bytes == 0


def test_table_only_tiles_run_only_where_measured(pkg):
    # The 8-wave 64x256, 128x128 and 64x128 split-K tiles measured ahead
    # only at the C3 shapes named here; the cost model would rank the first
    # at other skinny shapes where it measured slower, so only their
    # measured entries select them.
    home = {(16, 11008, 4096): (b"f16_nn_64x256x64_w2x4_s4_sk", 4),
            (128, 11008, 4096): (b"f16_nn_128x128x64_w2x4_s4_sk", 2),
            (16, 4096, 4096): (b"f16_nn_64x128x64_w2x4_s4_sk", 6),
            (128, 4096, 4096): (b"f16_nn_64x128x64_w2x4_s4_sk", 4),
            (128, 4096, 11008): (b"f16_nn_64x128x64_w2x4_s4_sk", 4),
            (16, 4096, 11008): (b"f16_nn_64x128x64_w2x4_s4_sk", 8),
            (192, 11008, 4096): (b"f16_nn_128x128x64_w2x4_s4_sk", 1)}
    names = [c.name for c in pkg.mfma_configs()]
    for shape, (name, splits) in home.items():
        assert name.decode() in names
        p = pkg.plan(pkg.make_desc(F16, F16, F16, *shape, 0))
        assert p.config_name == name and p.from_tuned_table
        assert p.splits == splits
    table_only = {name for name, _ in home.values()}
    # entries were timed on one matrix: a batch takes the model's pick
    for shape in home:
        p = pkg.plan(pkg.make_desc(F16, F16, F16, *shape, 0, batch=2))
        assert not p.from_tuned_table and p.config_name not in table_only
    for m in (8, 16, 24, 32, 48, 64, 128, 192, 256):
        for n, k in ((4096, 4096), (11008, 4096), (4096, 11008),
                     (11008, 11008), (512, 256), (8192, 4096)):
            if (m, n, k) in home:
                continue
            p = pkg.plan(pkg.make_desc(F16, F16, F16, m, n, k, 0))
            assert p.config_name not in table_only, (m, n, k)


def test_short_k_fills_the_cus(pkg):
    # Short K on a grid of few large tiles never overlaps its copies with
    # its MFMAs: the planner prefers more, smaller workgroups there
    # (2048x512x256: 32 workgroups of 256x128 measured 6.7 us, 64 of
    # 128x128 6.2 us; 512x512x256: 6.4 us against 4.3 us for 64 of 32x128
    # at one split; 256x11008x4096: 70.6 against 43.8 us).
    p = pkg.plan(pkg.make_desc(F16, F16, F16, 2048, 512, 256, 0))
    assert p.workgroups >= 64 and (p.tile_m, p.tile_n) != (256, 128)
    p = pkg.plan(pkg.make_desc(F16, F16, F16, 512, 512, 256, 0))
    assert p.config_name == b"f16_nn_32x128x64_w1x4_s4_sk" and p.splits == 1
    assert p.workgroups == 64 and p.workspace_bytes == 0
    p = pkg.plan(pkg.make_desc(F16, F16, F16, 256, 11008, 4096, 0))
    assert p.workgroups >= 128
    # a split grid keeps the overlapped pricing, so the split count is not
    # pushed past half the CUs (W8A16 96x2048x2048: x4 16.7 us, x8 20.4 us)
    p = pkg.plan(pkg.make_desc(F16, I8, F16, 96, 2048, 2048, 0,
                               has_scale=True))
    assert p.splits == 4


def test_planner_stream_k(pkg):
    # W8A16 192 x 11008 x 11008 on 128x256 tiles: 86 tiles for 256 CUs.
    # Stream-K runs (equal runs of (tile, K stage) pairs) measured fastest
    # here; the measured entry selects them.
    m, n, k = 192, 11008, 11008
    p = pkg.plan(pkg.make_desc(F16, I8, F16, m, n, k, 0, has_scale=True))
    assert p.stream_k_steps > 0 and p.from_tuned_table
    assert p.config_name.endswith(b"_sk")
    ks = k // p.tile_k
    tiles = -(-m // p.tile_m) * (n // p.tile_n)
    run = p.stream_k_steps
    assert p.workgroups == -(-tiles * ks // run) <= 256
    layers = max((t * ks + ks - 1) // run - t * ks // run + 1
                 for t in range(tiles))
    assert p.splits == layers > 1
    assert p.workspace_bytes == 256 * 1024 + layers * m * n * 4
    # Not ranked by the model (it won only where K is long): the C5 and C3
    # skinny shapes keep their split counts.
    for d in (pkg.make_desc(F16, I8, F16, 512, 11008, 4096, 0, has_scale=True),
              pkg.make_desc(F16, F16, F16, 192, 11008, 4096, 0),
              pkg.make_desc(F16, F16, F16, 16, 4096, 4096, 0)):
        assert pkg.plan(d).stream_k_steps == 0
    # batch > 1 never runs stream-K
    d = pkg.make_desc(F16, I8, F16, m, n, k, 0, has_scale=True)
    d.batch = 2
    assert pkg.plan(d).stream_k_steps == 0


# Argument validation: every call below fails on the host, so no GPU is needed.
FAKE = 0x10000  # 64 KiB aligned, never dereferenced


def call_f16(lib, a=FAKE, b=FAKE, c=FAKE, m=64, n=64, k=64, lda=64, ldb=64,
             ldc=64, flags=0):
    return lib.iree_mi355x_matmul_f16(a, b, c, m, n, k, lda, ldb, ldc, flags,
                                      None, 0, None)


def test_matmul_argument_errors(pkg):
    lib = pkg.library()
    assert call_f16(lib, m=-1) == pkg.INVALID_ARGUMENT
    assert call_f16(lib, a=None) == pkg.INVALID_ARGUMENT
    assert call_f16(lib, c=None) == pkg.INVALID_ARGUMENT
    assert call_f16(lib, lda=32) == pkg.INVALID_ARGUMENT
    assert call_f16(lib, ldc=63) == pkg.INVALID_ARGUMENT
    assert call_f16(lib, flags=0x80) == pkg.INVALID_ARGUMENT
    assert "unknown flag" in pkg.last_error()
    assert call_f16(lib, a=FAKE + 1) == pkg.MISALIGNED
    assert call_f16(lib, c=FAKE + 1, flags=pkg.OUT_F32) == pkg.MISALIGNED
    assert call_f16(lib, m=1 << 31) == pkg.UNSUPPORTED
    # empty output: a no-op that succeeds without touching the device
    assert call_f16(lib, m=0) == pkg.OK
    assert call_f16(lib, n=0, a=None, b=None) == pkg.OK
    assert lib.iree_mi355x_matmul_i8(FAKE, FAKE, FAKE + 2, 8, 8, 8, 8, 8, 8, 0,
                                     None, 0, None) == pkg.MISALIGNED
    assert lib.iree_mi355x_matmul_i8(FAKE, FAKE, FAKE, 8, 8, 8, 8, 8, 8,
                                     pkg.OUT_F32, None, 0,
                                     None) == pkg.INVALID_ARGUMENT
    assert lib.iree_mi355x_w8a16_matmul(FAKE, FAKE, None, FAKE, 1, 64, 64, 64,
                                        64, 64, 0, None, 0,
                                        None) == pkg.INVALID_ARGUMENT


def test_attention_argument_errors(pkg):
    lib = pkg.library()
    att = lib.iree_mi355x_attention_f16
    assert att(FAKE, FAKE, FAKE, FAKE, 1, 1, 128, 128, 96, 0.1, 1,
               None) == pkg.UNSUPPORTED
    assert att(FAKE, FAKE, FAKE, FAKE, 1, 1, 128, 128, 128, float("nan"), 1,
               None) == pkg.INVALID_ARGUMENT
    assert att(FAKE + 8, FAKE, FAKE, FAKE, 1, 1, 128, 128, 128, 0.1, 1,
               None) == pkg.MISALIGNED
    assert att(FAKE, FAKE, FAKE, FAKE, 1, 1, 128, 128, 128, 0.1, 4,
               None) == pkg.INVALID_ARGUMENT
    assert att(None, FAKE, FAKE, FAKE, 1, 1, 128, 128, 128, 0.1, 1,
               None) == pkg.INVALID_ARGUMENT
    assert att(FAKE, FAKE, FAKE, FAKE, 0, 1, 128, 128, 128, 0.1, 1,
               None) == pkg.OK
    # one head's K / V past 4 GiB (32-bit copy offsets)
    assert att(FAKE, FAKE, FAKE, FAKE, 1, 1, 128, 1 << 24, 128, 0.1, 0,
               None) == pkg.UNSUPPORTED
    assert "4 GiB" in pkg.last_error()
    assert att(FAKE, FAKE, FAKE, FAKE, 1, 1, 1 << 24, 128, 128, 0.1, 0,
               None) == pkg.UNSUPPORTED
    assert "4 GiB" in pkg.last_error()


def test_dispatch_rejects_short_bindings(pkg):
    consts = pkg.matmul_constants(64, 64, 64, 64, 64, 64, 0)
    full = [64 * 64 * 2] * 3
    short = [64 * 64 * 2, 64 * 64 * 2 - 2, 64 * 64 * 2]
    assert pkg.call_export("matmul_f16", consts, [FAKE] * 3,
                           short) == pkg.INVALID_ARGUMENT
    assert "binding 1" in pkg.last_error()
    # transposed B is [N,K]: the same byte count here, a different span formula
    consts_t = pkg.matmul_constants(64, 32, 64, 64, 64, 32, pkg.B_TRANSPOSED)
    assert pkg.call_export("matmul_f16", consts_t, [FAKE] * 3,
                           [64 * 64 * 2, 32 * 64 * 2 - 2, 64 * 32 * 2]) \
        == pkg.INVALID_ARGUMENT
    assert pkg.call_export("matmul_i8", consts[:5], [FAKE] * 3,
                           full) == pkg.INVALID_ARGUMENT
    att = pkg.attention_constants(1, 2, 128, 128, 64, 0.125, 1)
    q = 1 * 2 * 128 * 64 * 2
    assert pkg.call_export("attention_f16", att, [FAKE] * 4,
                           [q, q, q - 2, q]) == pkg.INVALID_ARGUMENT


def general_args(pkg, **kw):
    """An iree_mi355x_attention_t over contiguous operands (FAKE pointers:
    only checks that fail before any launch may use it)."""
    b, h, hkv, sq, skv, d, dv = (kw.pop(n, dflt) for n, dflt in (
        ("batch", 1), ("heads", 2), ("kv_heads", 2), ("seq_q", 64),
        ("seq_kv", 64), ("head_dim", 32), ("head_dim_v", 48)))
    a = pkg.AttentionArgs(q=FAKE, k=FAKE, v=FAKE, o=FAKE, batch=b, heads=h,
                          kv_heads=hkv, seq_q=sq, seq_kv=skv, head_dim=d,
                          head_dim_v=dv, scale=0.5, flags=0)
    a.strides.q[:] = [h * sq * d, sq * d, d]
    a.strides.k[:] = [hkv * skv * d, skv * d, d]
    a.strides.v[:] = [hkv * skv * dv, skv * dv, dv]
    a.strides.o[:] = [h * sq * dv, sq * dv, dv]
    for key, val in kw.items():
        setattr(a, key, val)
    return a


def test_general_attention_argument_errors(pkg):
    lib = pkg.library()

    def call(**kw):
        return lib.iree_mi355x_attention(ctypes.byref(general_args(pkg, **kw)),
                                         None)

    assert lib.iree_mi355x_attention(None, None) == pkg.INVALID_ARGUMENT
    assert call(flags=0x8) == pkg.INVALID_ARGUMENT
    assert "unknown flag" in pkg.last_error()
    # the MASK flag and the mask pointer go together
    assert call(flags=pkg.ATTENTION_MASK) == pkg.INVALID_ARGUMENT
    assert call(mask=FAKE) == pkg.INVALID_ARGUMENT
    assert "disagree" in pkg.last_error()
    assert call(head_dim=257) == pkg.UNSUPPORTED
    assert call(head_dim_v=300) == pkg.UNSUPPORTED
    assert call(head_dim=0) == pkg.UNSUPPORTED
    assert call(heads=6, kv_heads=4) == pkg.INVALID_ARGUMENT
    assert call(scale=float("inf")) == pkg.INVALID_ARGUMENT
    assert call(seq_q=-1) == pkg.INVALID_ARGUMENT
    assert call(batch=70000) == pkg.UNSUPPORTED
    assert call(q=None) == pkg.INVALID_ARGUMENT
    a = general_args(pkg, flags=pkg.ATTENTION_MASK, mask=FAKE)
    a.mask_strides[:] = [0, 0, -64, 1]
    assert lib.iree_mi355x_attention(ctypes.byref(a), None) \
        == pkg.INVALID_ARGUMENT
    assert "negative stride" in pkg.last_error()
    a = general_args(pkg)
    a.strides.o[2] = 47  # below head_dim_v
    assert lib.iree_mi355x_attention(ctypes.byref(a), None) \
        == pkg.INVALID_ARGUMENT
    # element alignment: f16 operands on 2 bytes, an f32 o on 4
    assert call(q=FAKE + 1) == pkg.MISALIGNED
    assert call(o=FAKE + 2, flags=pkg.ATTENTION_OUT_F32) == pkg.MISALIGNED
    assert call(mask=FAKE + 1, flags=pkg.ATTENTION_MASK) == pkg.MISALIGNED
    # nothing to write: succeeds without touching a device
    assert call(batch=0) == pkg.OK
    assert call(seq_q=0) == pkg.OK
    assert call(head_dim_v=0) == pkg.OK
    # the strict entry points keep their contract: head dims 64 / 128
    assert lib.iree_mi355x_attention_f16(FAKE, FAKE, FAKE, FAKE, 1, 1, 64, 64,
                                         96, 0.1, 0, None) == pkg.UNSUPPORTED


def test_general_attention_dispatch_bindings(pkg):
    # the 41-word form: head_dim_v, mask strides and the mask binding are
    # all checked against the bindings before any launch
    b, h, sq, skv, d, dv = 2, 3, 40, 50, 24, 40
    flags = pkg.ATTENTION_MASK | pkg.ATTENTION_OUT_F32
    row_mask = [0, 0, skv, 1]  # one [Sq, Skv] mask for every (batch, head)
    att = pkg.attention_constants(b, h, sq, skv, d, 0.5, flags,
                                  head_dim_v=dv, mask_strides=row_mask)
    assert len(att) == 41
    q = b * h * sq * d * 2
    kk = b * h * skv * d * 2
    vv = b * h * skv * dv * 2
    o = b * h * sq * dv * 4
    m = sq * skv * 2
    ok = [q, kk, vv, o, m]
    st, need = pkg.call_export("attention_f16", att, [FAKE] * 5, ok,
                               query=True)
    assert st == pkg.OK and need == 0, pkg.last_error()
    for i in range(5):
        short = list(ok)
        short[i] -= 2
        assert pkg.call_export("attention_f16", att, [FAKE] * 5, short,
                               query=True)[0] == pkg.INVALID_ARGUMENT
        assert f"binding {i}" in pkg.last_error()
    # a mask needs the 41-word form and its binding
    assert pkg.call_export("attention_f16", att, [FAKE] * 4, ok[:4],
                           query=True)[0] == pkg.INVALID_ARGUMENT
    short_form = pkg.attention_constants(b, h, sq, skv, d, 0.5,
                                         pkg.ATTENTION_MASK)
    assert pkg.call_export("attention_f16", short_form, [FAKE] * 5, ok,
                           query=True)[0] == pkg.INVALID_ARGUMENT
    assert "41-word" in pkg.last_error()


def test_batch_dispatch_rejects_short_bindings(pkg):
    """batch_matmul_f16 export: every binding, the batched spans included,
    is checked before anything launches."""
    z, m, n, k = 3, 64, 32, 16
    consts = pkg.batch_matmul_constants(m, n, k, k, n, n, 0, z, m * k, k * n,
                                        m * n, pkg.ACT_RELU, True, True, n, m * n)
    full = [z * m * k * 2, z * k * n * 2, z * m * n * 2, n * 2, z * m * n * 2]
    for i in range(5):
        short = list(full)
        short[i] -= 2
        assert pkg.call_export("batch_matmul_f16", consts, [FAKE] * 5,
                               short) == pkg.INVALID_ARGUMENT, i
    # fewer bindings than the epilogue bits announce
    assert pkg.call_export("batch_matmul_f16", consts, [FAKE] * 4,
                           full[:4]) == pkg.INVALID_ARGUMENT
    # too few constants
    assert pkg.call_export("batch_matmul_f16", consts[:20], [FAKE] * 5,
                           full) == pkg.INVALID_ARGUMENT


def test_batch_matmul_argument_checks(pkg):
    lib = pkg.library()
    f = lib.iree_mi355x_batch_matmul_f16
    # negative batch, batch over the grid limit, outputs that overlap
    assert f(FAKE, FAKE, FAKE, -1, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0, None,
             None, 0, None) == pkg.INVALID_ARGUMENT
    assert f(FAKE, FAKE, FAKE, 70000, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0, None,
             None, 0, None) == pkg.UNSUPPORTED
    assert f(FAKE, FAKE, FAKE, 2, 8, 8, 8, 8, 8, 8, 64, 64, 32, 0, None,
             None, 0, None) == pkg.INVALID_ARGUMENT
    e = pkg.Epilogue()
    e.activation = 7
    assert f(FAKE, FAKE, FAKE, 2, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0,
             ctypes.byref(e), None, 0, None) == pkg.INVALID_ARGUMENT
    e.activation = pkg.ACT_GELU_TANH
    e.multiplier = FAKE + 1
    assert f(FAKE, FAKE, FAKE, 2, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0,
             ctypes.byref(e), None, 0, None) == pkg.MISALIGNED
    e.multiplier = FAKE
    e.ld_multiplier = 4
    assert f(FAKE, FAKE, FAKE, 2, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0,
             ctypes.byref(e), None, 0, None) == pkg.INVALID_ARGUMENT
    # batch 0 is a no-op
    assert f(FAKE, FAKE, FAKE, 0, 8, 8, 8, 8, 8, 8, 64, 64, 64, 0, None,
             None, 0, None) == pkg.OK


def test_batch_planner_and_workspace(pkg):
    # batch spreads work over the CUs: fewer K splits than batch 1
    d1 = pkg.make_desc(0, 0, 0, 16, 4096, 4096, 0)
    d8 = pkg.make_desc(0, 0, 0, 16, 4096, 4096, 0, batch=8)
    p1, p8 = pkg.plan(d1), pkg.plan(d8)
    assert p8.family == pkg.FAMILY_MFMA and p8.splits < p1.splits
    assert p8.workgroups >= p1.workgroups
    # one split per tile stores directly: no workspace
    d32 = pkg.make_desc(0, 0, 0, 16, 4096, 4096, 0, batch=32)
    p32 = pkg.plan(d32)
    assert p32.family == pkg.FAMILY_MFMA and p32.splits == 1
    assert p32.workspace_bytes == 0
    lib = pkg.library()
    w1 = lib.iree_mi355x_batch_matmul_workspace_bytes(1, 1, 4096, 4096, 0)
    w4 = lib.iree_mi355x_batch_matmul_workspace_bytes(4, 1, 4096, 4096, 0)
    assert w1 == pkg.plan(pkg.make_desc(0, 0, 0, 1, 4096, 4096, 0)).workspace_bytes
    assert w4 > 64 * 1024 and w1 > 64 * 1024


# ------------------------------------------------------ transposed A ----

def test_transposed_a_planning(pkg):
    """A stored [K, M]: exact tiles take a transposed-A MFMA configuration of
    the same B form; ragged, skinny or misaligned shapes take the general
    kernel (never the GEMV, which streams A by rows)."""
    AT, BT = pkg.A_TRANSPOSED, pkg.B_TRANSPOSED
    for flags, form in ((AT, pkg.B_FORM_NN), (AT | BT, pkg.B_FORM_TN)):
        p = pkg.plan(pkg.make_desc(F16, F16, F16, 4096, 4096, 4096, flags))
        assert p.family == pkg.FAMILY_MFMA
        cfg = pkg.mfma_configs()[p.config_index]
        assert cfg.a_transposed and cfg.b_form == form
        assert pkg.plan(pkg.make_desc(F16, F16, F16, 64, 128, 96,
                                      flags)).family == pkg.FAMILY_GENERAL
        assert pkg.plan(pkg.make_desc(F16, F16, F16, 2, 4096, 4096,
                                      flags)).family == pkg.FAMILY_GENERAL
    # f32 output has transposed-A tiles too
    p = pkg.plan(pkg.make_desc(F16, F16, pkg.ELEM_F32, 512, 512, 512, AT))
    assert p.family == pkg.FAMILY_MFMA
    assert pkg.mfma_configs()[p.config_index].a_transposed
    # a plain-A dispatch never takes a transposed-A configuration
    for m, n, k in ((4096, 4096, 4096), (512, 512, 512), (256, 256, 128)):
        for flags in (0, BT):
            p = pkg.plan(pkg.make_desc(F16, F16, F16, m, n, k, flags))
            assert not pkg.mfma_configs()[p.config_index].a_transposed


def test_config_layout_flags(pkg):
    lib = pkg.library()
    cfgs = pkg.mfma_configs()
    assert any(c.a_transposed for c in cfgs)
    for c in cfgs:
        lf = lib.iree_mi355x_mfma_config_layout_flags(c.index)
        assert bool(lf & pkg.B_TRANSPOSED) == (c.b_form == pkg.B_FORM_TN)
        assert bool(lf & pkg.A_TRANSPOSED) == ("at_" in c.name)
        if c.a_transposed:
            assert c.a_elem == F16 and c.tile_m >= 128
    assert lib.iree_mi355x_mfma_config_layout_flags(len(cfgs)) == -1
    assert lib.iree_mi355x_mfma_config_layout_flags(-1) == -1


def test_transposed_a_argument_checks(pkg):
    lib = pkg.library()
    AT = pkg.A_TRANSPOSED
    # A [K, M] needs lda >= M (here M = 64 > lda = 32), not lda >= K
    assert call_f16(lib, flags=AT, lda=32) == pkg.INVALID_ARGUMENT
    # integer and W8A16 entry points take no transposed A
    assert lib.iree_mi355x_matmul_i8(FAKE, FAKE, FAKE, 8, 8, 8, 8, 8, 8, AT,
                                     None, 0, None) == pkg.INVALID_ARGUMENT
    assert lib.iree_mi355x_w8a16_matmul(FAKE, FAKE, FAKE, FAKE, 1, 64, 64, 64,
                                        64, 64, AT, None, 0,
                                        None) == pkg.INVALID_ARGUMENT
    # a configuration and the layout flags must agree
    at_cfg = [c for c in pkg.mfma_configs()
              if c.a_transposed and c.b_form == pkg.B_FORM_NN][0]
    f = lib.iree_mi355x_matmul_mfma_config
    assert f(at_cfg.index, FAKE, FAKE, None, FAKE, 256, 256, 256, 256, 256,
             256, 0, None, 0, None) == pkg.UNSUPPORTED


def test_fast_path_pitch_limit(pkg):
    """A row pitch of 8 MiB or more would overflow the 32-bit lane offsets of
    the fast kernels' copy side: such operands are not fast-path eligible."""
    lib = pkg.library()
    cfg = [c for c in pkg.mfma_configs() if c.name == "f16_nn_128x128x64_w2x2_s4"][0]
    f = lib.iree_mi355x_matmul_mfma_config
    big = (1 << 22)  # f16 elements: an 8 MiB row
    assert f(cfg.index, FAKE, FAKE, None, FAKE, 128, 128, 64, big, 128, 128, 0,
             None, 0, None) == pkg.UNSUPPORTED
    assert f(cfg.index, FAKE, FAKE, None, FAKE, 128, 128, 64, 128, big, 128, 0,
             None, 0, None) == pkg.UNSUPPORTED


# ------------------------------------------------------ kernel resources ----

def test_kernel_registry_without_device(pkg):
    """Every compiled kernel is listed with the exports that may launch it;
    every export has kernels, and every MFMA configuration is one of them."""
    ks = pkg.kernel_resources(device=False)
    names = [k["name"] for k in ks]
    assert len(names) == len(set(names)) == pkg.library().iree_mi355x_kernel_count()
    for cfg in pkg.mfma_configs():
        # a column split launches two listed kernels
        parts = column_split_parts(cfg.name) if "+" in cfg.name else [cfg.name]
        assert all(part in names for part in parts)
    for export in pkg.export_names():
        assert any(export in k["exports"] for k in ks), export
    by = {k["name"]: k for k in ks}
    assert by["general_i8"]["exports"] == ["matmul_i8"]
    assert set(by["gemv_f16_r1"]["exports"]) == {"matmul_f16", "batch_matmul_f16"}
    assert by["gemv_w8a16_r4"]["exports"] == ["w8a16_matmul"]
    assert by["runtime_fill"]["exports"] == []
    assert all(k["threads"] in (256, 512) for k in ks)
    assert "vgprs" not in by["general_i8"]       # needs a device
    lib = pkg.library()
    r = pkg.KernelResources()
    assert lib.iree_mi355x_kernel_resources(len(ks), ctypes.byref(r)) == \
        pkg.INVALID_ARGUMENT


def test_export_attributes_cover_mfma_configs(pkg):
    """Every export's static LDS / thread attributes cover the MFMA
    configurations it may launch (the GPU tests check equality against all
    of its kernels as loaded)."""
    lib = pkg.executable_library()
    names = pkg.export_names()
    by_name = {k["name"]: k for k in pkg.kernel_resources(device=False)}
    for cfg in pkg.mfma_configs():
        for export in by_name[cfg.name.split("+")[0]]["exports"]:
            attrs = lib.exports.attrs[names.index(export)]
            assert attrs.lds_bytes >= cfg.lds_bytes, (export, cfg.name)
            assert attrs.threads >= cfg.threads, (export, cfg.name)


def test_dispatch_binding_spans_do_not_wrap(pkg):
    """Binding sizes computed from caller constants are overflow-checked: an
    ld or extent whose byte span wraps int64 is rejected before any launch
    instead of wrapping to a small size a short binding would pass."""
    big = 1 << 62
    # (M - 1) * lda overflows: 3 * 2^62
    consts = pkg.matmul_constants(4, 64, 64, big, 64, 64, 0)
    assert pkg.call_export("matmul_f16", consts, [FAKE] * 3,
                           [4096] * 3) == pkg.INVALID_ARGUMENT
    assert "binding 0" in pkg.last_error()
    # wraps to exactly 2^64 + small: (rows-1)*ld + cols = 2^63 - 1 + 1
    consts = pkg.matmul_constants(2, 1, 1, (1 << 63) - 1, 1, 1, 0)
    assert pkg.call_export("matmul_f16", consts, [FAKE] * 3,
                           [64] * 3) == pkg.INVALID_ARGUMENT
    # attention: batch * heads * seq * d * 2 past 2^64 from 32-bit constants
    att = pkg.attention_constants(0xFFFFFFFF, 0xFFFFFFFF, 0xFFFF, 0xFFFF, 128,
                                  0.125, 0)
    assert pkg.call_export("attention_f16", att, [FAKE] * 4,
                           [1 << 20] * 4) == pkg.INVALID_ARGUMENT
    # batch strides: (batch - 1) * stride * 2 overflows
    z, m, n, k = 3, 8, 8, 8
    consts = pkg.batch_matmul_constants(m, n, k, k, n, n, 0, z, 1 << 62, 0,
                                        m * n)
    assert pkg.call_export("batch_matmul_f16", consts, [FAKE] * 3,
                           [1 << 20] * 3) == pkg.INVALID_ARGUMENT


def test_workspace_query_matches_dispatch_dry_run(pkg):
    """The workspace query is an upper bound of what the call needs, the
    M = 1 transposed-A row (planned as a GEMV) included; the dispatch
    dry run reports what the call would use."""
    lib = pkg.library()
    cases = [(1, 4096, 4096, pkg.A_TRANSPOSED, 1),
             (1, 4096, 4096, 0, 4096),
             (16, 4096, 11008, 0, 11008),
             (128, 11008, 4096, 0, 4096),
             (2048, 4096, 4096, 0, 4096)]
    for m, n, k, flags, lda in cases:
        q = lib.iree_mi355x_matmul_workspace_bytes(m, n, k, flags)
        consts = pkg.matmul_constants(m, n, k, lda, n, n, flags)
        a_bytes = (k * lda if flags & pkg.A_TRANSPOSED else m * lda) * 2
        st, need = pkg.call_export("matmul_f16", consts, [FAKE] * 3,
                                   [a_bytes, k * n * 2, m * n * 2],
                                   query=True)
        assert st == pkg.OK, pkg.last_error()
        assert need <= q, (m, n, k, flags, need, q)
        if flags & pkg.A_TRANSPOSED:
            assert need > 0  # runs as the GEMV, which needs a workspace
        qb = lib.iree_mi355x_batch_matmul_workspace_bytes(1, m, n, k, flags)
        assert need <= qb
