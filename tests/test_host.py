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
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(tao_\w+)\(",
                                 text, flags=re.M)))


def test_library_exports_every_header_symbol():
    lib = _hip.lib()
    declared = _header_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_hip.EXPORTED) == declared
    assert lib.tao_abi_version() == _hip.ABI_VERSION == 13


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


def test_prompt_attention_and_step_stamps_argument_checks():
    """tao_prompt_attention refuses a call whose window reaches before the
    call (a continuing prefill needs the state's ring), too few tile words
    and bad geometry, before any device work; tao_step_stamps refuses
    frames of fewer than 8 words and turns off with a null buffer."""
    lib = _hip.lib()
    cfg = _hip.StreamCfg(0, 512, 256, 8, 24, 2, 1, 2, 0)
    tok = _hip.Tokens()
    for name in ("q", "k", "v", "raw_q", "raw_k"):
        setattr(tok, name, 0x1000)          # never dereferenced: checks come first
    tok.tokens = 300
    fake = ctypes.c_void_p(0x2000)
    rc = lib.tao_prompt_attention(ctypes.byref(cfg), 1, 4, 128, ctypes.byref(tok), 1000,
                                  fake, 1 << 20, fake, None)
    assert rc < 0 and b"window" in lib.tao_last_error()
    rc = lib.tao_prompt_attention(ctypes.byref(cfg), 1, 4, 128, ctypes.byref(tok), 0,
                                  fake, 2, fake, None)
    assert rc < 0 and b"tiles_cap" in lib.tao_last_error()
    rc = lib.tao_prompt_attention(ctypes.byref(cfg), 1, 4, 96, ctypes.byref(tok), 0,
                                  fake, 1 << 20, fake, None)
    assert rc < 0 and b"geometry" in lib.tao_last_error()
    assert lib.tao_step_stamps(fake, 4, 7) < 0
    assert lib.tao_step_stamps(fake, 0, 64) < 0
    assert lib.tao_step_stamps(None, 0, 0) == 0 and lib.tao_step_stamps_count() == 0


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


def _reference_plan(cfg, layer, route_coarse, route_size, pos0, tokens, outputs):
    """Prefill plan written out from the schedule closed forms (checker for
    the library's tao_prefill_plan)."""
    group = cfg.coarse_group
    end = pos0 + tokens
    f0, f1 = schedule.fines_at(pos0, cfg), schedule.fines_at(end, cfg)
    plan_chunks = schedule.chunks(pos0, tokens, cfg)
    attn, reads, turns, chunk_epochs = [], [], [], []
    for start, width in plan_chunks:
        epoch = schedule.fines_at(start, cfg)
        chunk_epochs.append(epoch)
        if outputs:
            key_start = start - schedule.local_len_at(start, cfg)
            for qs in range(start, start + width, 256):
                attn += [qs - pos0, min(256, start + width - qs), key_start]
    first_epoch = 0
    if f1 >= 1:
        first_epoch = max(min([e for e in chunk_epochs if e >= 1] + [f1]), 1)
        if not outputs:
            first_epoch = f1
    slot, slot_m = 0, route_size
    route = (route_coarse, route_size)
    last_turn = None
    for (start, width), epoch in zip(plan_chunks, chunk_epochs):
        for sub, count, refresh in schedule.sub_chunks(start, width, layer, cfg):
            if epoch == 0:
                if outputs:
                    for qs in range(sub, sub + count, 32):
                        reads += [qs - pos0, min(32, sub + count - qs), 0, 0, 0, 0, 0, 0]
                continue
            if refresh:
                completed, pending = divmod(epoch, group)
                coarse, _, selected = schedule.routed_counts(completed, pending, cfg)
                last_turn = (sub, epoch, completed, pending, coarse, selected)
                if outputs:
                    turns += [sub - pos0, epoch - first_epoch, completed, pending, coarse,
                              selected, len(turns) // 8 + 1, 0]
                    slot, slot_m = len(turns) // 8, selected
                route = (coarse, selected)
            if outputs:
                for qs in range(sub, sub + count, 32):
                    reads += [qs - pos0, min(32, sub + count - qs), slot, slot_m,
                              epoch - first_epoch, (epoch // group) * group, 1,
                              epoch // group]
    if not outputs and last_turn is not None:
        sub, epoch, completed, pending, coarse, selected = last_turn
        first_epoch = min(first_epoch, epoch)
        turns = [sub - pos0, epoch - first_epoch, completed, pending, coarse, selected, 1, 1]
    elif turns:
        turns[-1] = 1
    n_epochs = f1 - first_epoch + 1 if f1 >= 1 else 0
    writes = [cfg.fine_tokens * f for f in range(f0, f1)]
    keep = min(tokens, cfg.serve_limit)
    header = [0] * _hip.PLAN_HEADER
    header[:13] = [pos0, len(attn) // 3, len(writes), f0, f0 // group,
                   f1 // group - f0 // group, first_epoch, n_epochs, len(turns) // 8,
                   len(reads) // 8, tokens - keep, keep, end - keep]
    history = sum(1 for e in chunk_epochs if e)
    read_pages = [e // group for e in chunk_epochs if e // group >= 1] if outputs else []
    coarse_range = ((min(read_pages), max(read_pages) - min(read_pages) + 1)
                    if read_pages else (0, 0))
    info = [None, n_epochs, len(turns) // 8, route[0], route[1], f1 // group + 1, history,
            len(chunk_epochs), *coarse_range]
    return header + attn + writes + turns + reads, info


def test_native_prefill_plan_matches_closed_forms():
    """tao_prefill_plan (host code in the library) against the plan written
    out from the schedule closed forms, over positions, widths, layers,
    carried routes and both modes."""
    import numpy as np
    lib = _hip.lib()
    cfg = index_only_page_memo()
    cases = 0
    for layer in (0, 1, 5):
        scfg = _hip.StreamCfg(layer, cfg.local_keep, cfg.fine_tokens, cfg.coarse_group,
                              cfg.route_period, cfg.layer_stagger, cfg.budget_root_scale,
                              cfg.budget_offset, 0)
        for pos0 in (0, 100, 767, 768, 769, 1000, 2050, 5000, 131072):
            for tokens in (0, 1, 5, 24, 255, 256, 300, 800, 2048, 6000):
                f = schedule.fines_at(pos0, cfg)
                routes = [(0, 0)] if f == 0 else [(1, 3), (4, 14)]
                for rc, rs in routes:
                    for outputs in (True, False):
                        want, want_info = _reference_plan(cfg, layer, rc, rs, pos0, tokens,
                                                          outputs)
                        info = (ctypes.c_int64 * 10)()
                        args = (ctypes.byref(scfg), pos0, tokens, rc, rs, int(outputs))
                        assert lib.tao_prefill_plan(*args, None, 0, info) == 0
                        assert info[0] == len(want)
                        got = np.zeros(info[0], dtype=np.int64)
                        assert lib.tao_prefill_plan(*args, got.ctypes.data, info[0], info) == 0
                        assert got.tolist() == want, (layer, pos0, tokens, rc, rs, outputs)
                        assert list(info)[1:] == want_info[1:]
                        cases += 1
    assert cases > 400
    small = (ctypes.c_int64 * 10)()
    buf = np.zeros(4, dtype=np.int64)
    assert lib.tao_prefill_plan(ctypes.byref(scfg), 0, 300, 0, 0, 1, buf.ctypes.data, 4,
                                small) < 0


def test_native_train_plan_matches_read_training_tiling():
    """tao_train_plan against read_training's tiling written out from the
    closed forms (tao_stream.py:668-787): 256-token tiles with local keys
    from max(0, 256 t - 512), t - 2 visible fines, the routed counts of each
    tile's epoch, every query routing itself, no ring append."""
    import numpy as np
    from tao_attention import training
    g = O.Geometry()
    for cfg in (TaoConfig(), index_only_page_memo()):
        for tokens in (0, 1, 255, 700, 768, 769, 1000, 1024, 2900, 8192, 16385):
            plan, info = training.plan(cfg, tokens)
            n_tiles = -(-tokens // 256)
            vmax = max(0, n_tiles - 3)
            h = plan[:16]
            assert h[13] == 1 and h[8] == 0 and h[0] == 0
            assert (h[10], h[11], h[12]) == (tokens, 0, tokens)
            assert h[2] == vmax and h[5] == vmax // 8
            assert (h[6], h[7]) == ((1, vmax) if vmax else (0, 0))
            assert info["fines"] == vmax and info["qsel_words"] == (vmax + 31) // 32
            off = 16
            attn = plan[off:off + 3 * h[1]].reshape(-1, 3)
            off += 3 * h[1]
            want = [(s, min(256, tokens - s), max(0, s - 512)) for s in range(0, tokens, 256)]
            assert [tuple(r) for r in attn.tolist()] == want
            assert plan[off:off + h[2]].tolist() == [256 * f for f in range(vmax)]
            off += h[2]
            reads = plan[off:].reshape(-1, 8)
            assert len(reads) == h[9] and off + 8 * h[9] == len(plan) == info["length"]
            starts = []
            for first, n, coarse, m, erel, split, on, cpages in reads.tolist():
                starts.append(first)
                visible = max(0, first // 256 - 2)
                assert n == min(32, tokens - first, 256 - first % 256)
                if not visible:
                    assert (coarse, m, erel, split, on, cpages) == (0, 0, 0, 0, 0, 0)
                    continue
                c, _, sel = g.routed_counts(visible // 8, visible % 8)
                assert (coarse, m, erel, split, on, cpages) == (
                    c, sel, visible - 1, (visible // 8) * 8, 1, visible // 8)
            assert starts == list(range(0, tokens, 32))


def test_graph_stat_layout_matches_header():
    """The Python view of the driver's epoch counters uses the header's enums."""
    text = open(os.path.join(ROOT, "include", "tao_memory.h")).read()
    reasons = re.findall(r"TAO_GRAPH_(\w+) = (\d+),", text)
    names = {name.lower(): int(value) for name, value in reasons}
    assert [names[r] for r in _hip.GRAPH_REASONS] == list(range(len(_hip.GRAPH_REASONS)))
    assert int(re.search(r"TAO_GRAPH_REASONS = (\d+)", text).group(1)) == len(_hip.GRAPH_REASONS)
    stats = dict(re.findall(r"(TAO_GS_\w+) = (\d+)", text))
    assert int(stats["TAO_GS_REASON0"]) + len(_hip.GRAPH_REASONS) == _hip.GRAPH_STATS
    assert (int(stats["TAO_GS_LAST_ACTION"]), int(stats["TAO_GS_LAST_REASON"])) == (10, 11)
    assert int(stats["TAO_GS_EPOCH_VERSION"]) == 8 and int(stats["TAO_GS_WARM"]) == 9
