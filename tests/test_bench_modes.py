"""bench.py's host-only mode: the encoder throughput line, byte-identical to the oracle (run_encode raises
otherwise), and the JSON fields the report relies on."""
import argparse

import bench


def test_encode_mode_line_cpu():
    line = bench.run_encode(argparse.Namespace())
    assert line["byte_identical_to_oracle"] is True
    assert line["unit"] == "M weights/s" and line["value"] > 0
    assert line["cpu_baseline"]["kind"] == "port" and line["cpu_baseline"]["cores"] == 1
    assert line["speedup"] > 0
