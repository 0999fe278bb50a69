"""SPKV2_TUNE_DB: a later process reuses the measured tile choices, hybrid
schedules included (their split is stored as 1000 + slices per remaining
tile)."""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

# one conv with enough tiles for the hybrid schedule; prints its kernel name
# and a checksum of its output
CHILD = r"""
import json, sys
sys.path.insert(0, %r)
import numpy as np
from spinnv2_amd.runtime import Model
from spinnv2_amd.spk import models, write_spk
g = models.single_conv(4, 16, 63, 67, 200, 3, 1, 1, act="Relu")
x = models.make_input(g.tensors[g.inputs[0]].shape, 11)
with Model(write_spk(g, "mi355x")) as m:
    m.set_input(0, x)
    m.run()
    y = m.get_output(0)
    print(json.dumps({"name": m.kernel_name(0), "sum": float(np.abs(y).sum())}))
""" % str(ROOT)


def _child(db: Path) -> dict:
    env = dict(os.environ, SPKV2_TUNE_DB=str(db))
    for k in ("SPKV2_CONV_CFG", "SPKV2_CONV_SPLITK", "SPKV2_CONV_HYBRID", "SPKV2_CONV_TUNE"):
        env.pop(k, None)
    out = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=100)
    assert out.returncode == 0, out.stderr[-2000:]
    return json.loads(out.stdout.strip().splitlines()[-1])


NETWORK_CHILD = r"""
import hashlib, json, sys
sys.path.insert(0, %r)
from spinnv2_amd.runtime import Model
from spinnv2_amd.spk import models, write_spk
g = models.resnet(101, 1)
x = models.make_input(g.tensors[g.inputs[0]].shape, 5)
with Model(write_spk(g, "mi355x")) as m:
    m.set_input(0, x)
    m.run()
    y = m.get_output(0)
    names = [m.kernel_name(n.id) for n in g.nodes if n.op_type in ("Conv", "Gemm")]
print(json.dumps({"sha": hashlib.sha256(y.tobytes()).hexdigest(), "names": names}))
""" % str(ROOT)


def test_benchmark_network_is_bit_reproducible_across_processes(gpu):
    """The committed tune table (spinnv2_amd/lib/mi355x.tune) fixes the tile
    and split-K choice of every ResNet-101 layer, so two fresh processes
    without a tune DB of their own pick the same kernels and produce the
    same logits bit for bit."""
    assert (ROOT / "spinnv2_amd" / "lib" / "mi355x.tune").stat().st_size > 0
    env = dict(os.environ)
    for k in ("SPKV2_TUNE_DB", "SPKV2_TUNE_TABLE", "SPKV2_CONV_CFG", "SPKV2_CONV_SPLITK", "SPKV2_CONV_HYBRID",
              "SPKV2_CONV_TUNE"):
        env.pop(k, None)
    runs = []
    for _ in range(2):
        out = subprocess.run([sys.executable, "-c", NETWORK_CHILD], env=env, capture_output=True, text=True,
                             timeout=100)
        assert out.returncode == 0, out.stderr[-2000:]
        runs.append(json.loads(out.stdout.strip().splitlines()[-1]))
    assert runs[0]["names"] == runs[1]["names"]
    assert runs[0]["sha"] == runs[1]["sha"]


def test_tune_db_reuses_hybrid_choice(gpu, tmp_path):
    db = tmp_path / "tune.db"
    first = _child(db)
    lines = db.read_text().split("\n")
    conv = [ln for ln in lines if ln.startswith("conv|")]
    assert len(conv) == 1, lines
    key, cfg, _ = conv[0].split()
    # replace the measured choice with a hybrid schedule of 4 slices
    db.write_text(f"{key} {cfg} 1004\n")
    second = _child(db)
    assert ",dp=" in second["name"], second
    assert abs(second["sum"] - first["sum"]) <= 1e-4 * first["sum"]
    assert db.read_text() == f"{key} {cfg} 1004\n"  # a hit stores nothing new
