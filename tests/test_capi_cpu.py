"""CPU-only checks of the product boundary: libesm_gfx950.so loads and exports
every entry point include/esm_gfx950.h declares; the host-side helpers that
need no GPU (RoPE tables) behave; no compute call is made."""
import os
import re

import numpy as np

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "esm_gfx950.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(esm_gfx950_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    import esm_gfx950 as eg
    assert declared_symbols() == sorted(eg.EXPORTED)


def test_library_exports_every_declared_symbol():
    import esm_gfx950 as eg
    lib = eg.load_library()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_rope_tables_match_reference_formula(oracle):
    import esm_gfx950 as eg
    for L, dh in ((1, 4), (250, 64), (1024, 64), (202, 16)):
        c, s = eg.rope_build_tables(L, dh)
        oc, os_ = oracle.rope_tables(L, dh)
        assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_product_does_not_reference_oracle():
    """The product sources never include, load or name the checker."""
    pkg = os.path.join(ROOT, "esm-cpp_amd")
    for dirpath, _, files in os.walk(pkg):
        if "_build" in dirpath or "lib" == os.path.basename(dirpath):
            continue
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "pyoracle" not in text and "liboracle" not in text and "libesmref" not in text, f


def test_attention_work_list_fits_its_metadata_region():
    """The per-XCD queues of the MFMA attention's work list are padded to the
    longest queue, which with few heads and one long sequence can reach 8x
    that sequence's tiles: the metadata region must be sized for that bound
    (esm_gfx950_batch_upload copies the list into it)."""
    import esm_gfx950 as eg
    from conftest import cu_from_lengths
    rs = np.random.default_rng(5)
    cases = [[1024], [1], [2048], [1024, 3], [300, 300, 7], [129] * 5, [4096, 1, 1, 1]]
    cases += [list(rs.integers(1, 1100, size=n)) for n in (1, 2, 3, 8, 31, 256)]
    for lengths in cases:
        cu = cu_from_lengths(lengths)
        for H in (1, 2, 3, 4, 5, 20, 40):
            for mfma in (True, False):
                items, cap = eg.attention_work_items(cu, H, mfma)
                assert items <= cap, (lengths, H, mfma, items, cap)
    # The case the bound was derived for: d = 128, H = 2, one 1024-token
    # sequence produces 64 items (8 queues padded to 8 tiles).
    items, cap = eg.attention_work_items(cu_from_lengths([1024]), 2, True)
    assert items == 64 and cap >= 64
