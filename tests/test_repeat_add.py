"""Closed-form replay of repeated sequential double adds (the exact top_p
replay of a tie group at the row maximum) against the literal loop, on the
CPU: tests/cpp/repeat_add_check.cpp, built by the package Makefile."""
import os
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "bin", "repeat_add_check")


def test_repeat_add_matches_literal_loop():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(REPO, "mlx-confucius4-tts_amd"),
                        "../tests/cpp/bin/repeat_add_check"], check=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout
