"""CPU checks of bench.py's contract: one GPU only, and the byte accounting behind
the roofline figure."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_headline_algorithmic_bytes():
    import bench
    # W3A4 [17408, 5120] batch 5, counted operand by operand: 3-bit codes, one fp16
    # scale per row and 128-column group, 4-bit activation codes, one fp16 activation
    # scale per token and group, fp32 outputs.
    codes = 17408 * 5120 * 3 // 8          # 33,423,360
    scales = 17408 * 40 * 2                 # 1,392,640
    acts = 5 * 5120 // 2 + 5 * 40 * 2       # 12,800 + 400
    outs = 5 * 17408 * 4                    # 348,160
    assert bench.algorithmic_bytes(17408, 5120, 5) == codes + scales + acts + outs == 35177360
    # W4, the down shape and one token change only the terms they name
    assert bench.algorithmic_bytes(5120, 17408, 1, wbits=4) == (
        5120 * 17408 // 2 + 5120 * 136 * 2 + 17408 // 2 + 136 * 2 + 5120 * 4)


def test_committed_traffic_is_withheld_when_the_kernel_source_changed(tmp_path, monkeypatch):
    """The roofline's traffic comes from a committed PMC summary; it is reported only
    while the headline kernel's source still has the digest that summary measured."""
    import bench
    digest = bench.headline_kernel_digest()
    summary = tmp_path / "summary.txt"
    for recorded, expect in ((digest, 35403459), ("0" * 16, None)):
        summary.write_text(f"kernel_avg_us = 9.6\ntraffic_bytes_per_launch = 35403459\n"
                           f"kernel_source_sha256 = {recorded}\n")
        monkeypatch.setattr(bench, "PROFILE", str(summary))
        profile = bench.committed_profile()
        assert profile["traffic"] == expect
        assert profile["source_matches"] == (expect is not None)
