"""Host logic and the C-ABI boundary (CPU only, no kernel launches)."""
import ctypes
import os
import re

import pytest
import torch

from oracle import tao_oracle as O
from tao_attention import TaoConfig, schedule
from tao_attention import _hip
from tao_attention.presets import index_only_page_memo

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_config_contract_errors():
    with pytest.raises(ValueError):
        TaoConfig(fine_writer="nope")
    with pytest.raises(TypeError):
        TaoConfig(fine_tokens=256.0)
    with pytest.raises(ValueError):
        TaoConfig(local_keep=500)
    with pytest.raises(ValueError):
        TaoConfig(route_period=0)
    with pytest.raises(ValueError):
        TaoConfig(layer_stagger=-1)
    cfg = index_only_page_memo(graph=True)
    assert TaoConfig(**cfg.export()) == cfg
    assert cfg.coarse_index_only and cfg.q1_page_normalization_memo
    assert cfg.q1_history_region_graph
    assert (cfg.serve_limit, cfg.first_fine, cfg.first_coarse, cfg.visibility_tiles) == (
        768, 768, 2560, 2)


def test_schedule_matches_oracle_closed_forms():
    cfg = index_only_page_memo()
    g = O.Geometry()
    for layer in (0, 1, 7):
        for p in range(0, 4000, 7):
            assert schedule.is_turn(p, layer, cfg) == g.is_turn(p, layer)
            assert schedule.next_turn(p, layer, cfg) == g.next_turn(p, layer)
    for completed in range(0, 70):
        for pending in range(0, 8):
            if completed or pending:
                assert schedule.routed_counts(completed, pending, cfg) == \
                    g.routed_counts(completed, pending)


def test_schedule_local_and_fines_follow_oracle_stream():
    """local_len_at / fines_at equal the oracle's explicit window bookkeeping."""
    cfg = index_only_page_memo()
    xs = [torch.zeros(1, 2000, 1, 4, dtype=torch.bfloat16) for _ in range(5)]
    fa = fb = torch.zeros(1, 4, 3)
    s = O.OracleStream(0)
    pos = 0
    for width in (100, 300, 256, 1, 1, 500, 77, 765):
        chunks = schedule.chunks(pos, width, cfg)
        assert sum(w for _, w in chunks) == width
        end = pos + width
        for start, w in chunks:
            assert start == s.position
            assert w == s.next_chunk(end - start)
            s.prefill(*(x[:, start:start + w] for x in xs), fa, fb, 0.5)
            assert schedule.local_len_at(s.position, cfg) == s.local[0].shape[1]
            assert schedule.fines_at(s.position, cfg) == len(s.fine_z)
            assert schedule.seals_in(start, w, cfg) == (
                schedule.fines_at(start + w, cfg) > schedule.fines_at(start, cfg))
        pos = end


def _header_functions():
    text = open(os.path.join(ROOT, "include", "tao_memory.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tao_\w+)\(",
                                 text, flags=re.M)))


def test_library_exports_every_header_symbol():
    lib = _hip.lib()
    declared = _header_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_hip.EXPORTED) == declared
    assert lib.tao_abi_version() == 2


def test_workspace_size_and_error_convention():
    lib = _hip.lib()
    small = lib.tao_workspace_bytes(1, 4, 64, 8, 0)
    large = lib.tao_workspace_bytes(1, 32, 128, 64, 16384)
    assert 0 < small < large
    st = _hip.StateDev()   # all-null: contract error, no launch
    rc = lib.tao_workspace_init(ctypes.byref(st), None)
    assert rc < 0
    with pytest.raises(ValueError):
        _hip.check(rc)


def test_product_has_no_oracle_or_cpu_path():
    pkg = os.path.join(ROOT, "tao-memory_amd", "tao_attention")
    for name in os.listdir(pkg):
        if name.endswith(".py"):
            text = open(os.path.join(pkg, name)).read()
            assert "oracle" not in text.replace("oracles", ""), name


def test_count_turns_closed_form():
    cfg = index_only_page_memo()
    for layer in (0, 1, 5, 40):
        for lo in (0, 700, 768, 769, 800, 1000):
            for hi in (lo, lo + 1, lo + 23, lo + 24, lo + 500, lo + 3000):
                brute = sum(1 for p in range(lo, hi) if schedule.is_turn(p, layer, cfg))
                assert schedule.count_turns(lo, hi, layer, cfg) == brute, (layer, lo, hi)
