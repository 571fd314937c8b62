"""The committed rocprof summaries bench.py reads traffic from: each names the traffic per
launch and the digest of the kernel sources it measured, and bench.py uses the traffic only
while the sources still hash to that digest (a kernel changed after its profile reports
traffic null)."""
import os
import re

import pytest

import bench

pytestmark = pytest.mark.filterwarnings("ignore")


@pytest.mark.parametrize("workload", sorted(bench.PMC_SUMMARY))
def test_summary_names_traffic_and_sources(workload):
    text = open(bench.PMC_SUMMARY[workload]).read()
    assert re.search(r"traffic_bytes_per_launch\s*=\s*[0-9]+", text), workload
    assert re.search(r"kernel_sources_sha256\s*=\s*[0-9a-f]{64}", text), workload
    for name in bench.PMC_SOURCES[workload]:
        assert os.path.exists(os.path.join(bench.ROOT, "polar_pack_amd", "csrc", name)), name


def test_traffic_only_for_the_measured_sources(tmp_path):
    src = bench.PMC_SOURCES["quad3b"]
    digest = bench.kernel_sources_sha256(src)
    good = tmp_path / "good.md"
    good.write_text(f"traffic_bytes_per_launch = 1234\n\nkernel_sources_sha256 = {digest}\n")
    assert bench.read_pmc_traffic(str(good), src) == 1234.0
    stale = tmp_path / "stale.md"
    stale.write_text(f"traffic_bytes_per_launch = 1234\n\nkernel_sources_sha256 = {'0' * 64}\n")
    assert bench.read_pmc_traffic(str(stale), src) is None
    unnamed = tmp_path / "unnamed.md"
    unnamed.write_text("traffic_bytes_per_launch = 1234\n")
    assert bench.read_pmc_traffic(str(unnamed), src) is None
    assert bench.read_pmc_traffic(str(unnamed)) == 1234.0
    assert bench.read_pmc_traffic(str(tmp_path / "missing.md"), src) is None


def test_digest_follows_every_source(tmp_path, monkeypatch):
    """Changing any one of the files changes the digest."""
    names = ["a.hip", "b.h"]
    csrc = tmp_path / "polar_pack_amd" / "csrc"
    csrc.mkdir(parents=True)
    (csrc / "a.hip").write_text("kernel a")
    (csrc / "b.h").write_text("header b")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    d0 = bench.kernel_sources_sha256(names)
    (csrc / "b.h").write_text("header b changed")
    d1 = bench.kernel_sources_sha256(names)
    (csrc / "a.hip").write_text("kernel a changed")
    d2 = bench.kernel_sources_sha256(names)
    assert len({d0, d1, d2}) == 3
