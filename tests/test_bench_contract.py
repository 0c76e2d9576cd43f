"""bench.py's host-side contract pieces that need no GPU: the one-GPU refusal and the rule that
`roofline.traffic` comes from the committed PMC summary only for the kernel sources it was
collected on."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_traffic_summary_is_used_only_for_its_kernel_sources(monkeypatch, tmp_path):
    summary = tmp_path / "traffic.md"
    summary.write_text("traffic_bytes_per_launch: 123\nkernel_sources_sha256: "
                       f"{bench.kernel_source_digest()}\n", encoding="utf-8")
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", summary)
    assert bench.profiled_traffic(64) == (123.0, None)
    value, note = bench.profiled_traffic(32)
    assert value is None and "batch 64" in note
    summary.write_text("traffic_bytes_per_launch: 123\nkernel_sources_sha256: 00\n",
                       encoding="utf-8")
    value, note = bench.profiled_traffic(64)
    assert value is None and "other kernel sources" in note
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", tmp_path / "absent.md")
    assert bench.profiled_traffic(64) == (None, "no traffic summary")


def test_committed_traffic_summary_names_a_digest_and_a_byte_count():
    text = (ROOT / "profiles" / "gemm_decode_w1_bs64_hbm_traffic.md").read_text(encoding="utf-8")
    keys = {line.split(":", 1)[0] for line in text.splitlines() if ":" in line}
    assert {"traffic_bytes_per_launch", "kernel_sources_sha256"} <= keys


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in json.loads(out.stdout.strip().splitlines()[-1])["error"]
