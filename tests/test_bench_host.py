"""Host-side logic of bench.py, on the CPU: the gate that lets a committed
counter profile into the bench line only for the kernel sources it was
measured on, the contiguous placements of the decode comparators, and the
refusal of more than one GPU."""

from __future__ import annotations

import json
import os
import subprocess
import sys
import types

import torch

import bench

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _tree(tmp_path, kernel_text="kernel A"):
    """A minimal tree: one kernel source, the ABI header and profiles/."""
    (tmp_path / "mini-llm-runtime_amd" / "csrc").mkdir(parents=True)
    (tmp_path / "include").mkdir()
    (tmp_path / "profiles").mkdir()
    (tmp_path / "mini-llm-runtime_amd" / "csrc" / "k.hip").write_text(kernel_text)
    (tmp_path / "include" / "mlr_attn.h").write_text("int f(void);\n")
    return tmp_path


def _write_traffic(tree, sha):
    (tree / "profiles" / "traffic.json").write_text(json.dumps(
        {"source": "profiles/x_traffic.md", "kernel_sources_sha256_16": sha,
         "decode_step_bytes": 123}))


def test_traffic_is_used_only_for_the_sources_it_was_measured_on(tmp_path, monkeypatch):
    tree = _tree(tmp_path)
    monkeypatch.setattr(bench, "REPO", str(tree))
    assert bench.measured_traffic() == (None, "profiles/traffic.json is absent")
    sha = bench.kernel_sources_hash()
    _write_traffic(tree, sha)
    traffic, source = bench.measured_traffic()
    assert traffic["decode_step_bytes"] == 123 and source == "profiles/x_traffic.md"
    # Any change to a kernel source or the header makes the profile stale.
    (tree / "mini-llm-runtime_amd" / "csrc" / "k.hip").write_text("kernel B")
    traffic, reason = bench.measured_traffic()
    assert traffic is None and "other kernel sources" in reason and sha in reason
    (tree / "mini-llm-runtime_amd" / "csrc" / "k.hip").write_text("kernel A")
    assert bench.measured_traffic()[0] is not None
    (tree / "include" / "mlr_attn.h").write_text("int f(int);\n")
    assert bench.measured_traffic()[0] is None


def test_kernel_sources_hash_depends_on_names_and_contents(tmp_path, monkeypatch):
    a = _tree(tmp_path / "a")
    b = _tree(tmp_path / "b")
    monkeypatch.setattr(bench, "REPO", str(a))
    ha = bench.kernel_sources_hash()
    monkeypatch.setattr(bench, "REPO", str(b))
    assert bench.kernel_sources_hash() == ha  # same names, same bytes
    os.rename(b / "mini-llm-runtime_amd" / "csrc" / "k.hip",
              b / "mini-llm-runtime_amd" / "csrc" / "k2.hip")
    assert bench.kernel_sources_hash() != ha


def test_contiguous_tables_place_each_sequence_in_consecutive_blocks():
    lens = [1, 16, 17, 300, 33]
    width = 20
    wl = types.SimpleNamespace(context_lens=torch.tensor(lens),
                               block_tables=torch.full((len(lens), width), -1))
    bt_seq, slots_seq, bt_flat, ctx_flat = bench.contiguous_tables(wl, torch.device("cpu"))
    start = 0
    for b, n in enumerate(lens):
        need = -(-n // 16)
        assert bt_seq[b, :need].tolist() == list(range(start, start + need))
        assert (bt_seq[b, need:] == -1).all()
        # The new token's slot is that of position n - 1 in this table.
        assert int(slots_seq[b]) == (start + (n - 1) // 16) * 16 + (n - 1) % 16
        start += need
    total = sum(lens)
    assert int(ctx_flat) == total
    assert bt_flat.tolist() == [list(range(-(-total // 16)))]


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def test_a_distributed_launch_is_refused():
    res = subprocess.run([sys.executable, os.path.join(REPO, "bench.py")],
                         capture_output=True, text=True, timeout=60,
                         env={**os.environ, "WORLD_SIZE": "4"})
    assert res.returncode == 2 and "one GPU" in res.stderr
