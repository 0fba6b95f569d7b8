"""The device router's register nth_element (mimo-prismwing_amd/csrc/pw_select_wave.h) on the CPU:
tests/select_wave_check.cpp runs the header's algorithm with a 64-lane wave emulated by 64 threads
and compares the whole row it leaves with the serial libc++ nth_element restatement (pw_topk.h,
pinned by the reference's golden top-k orders pw0063 / pw0157) for random, tied, equal, sorted and
one-high rows of 9 to 1024 entries at nth 7 (the router's top-8) and at n - 1 or a random position;
and the whole routed row (select_route_row: corrected scores, top 8, boundary, renormalised weights
on lanes 0..7) against the host routing (noaux_route_row) bit for bit, with ties and a non-finite bias;
and the fast set (fast_top8_set), which must decide exactly the rows with finite values and an untied
boundary, and then give the host's eight ids.
(The emulation costs about a tenth of a second per row; the full sweep, `select_wave_check 25`, ran
6,135 rows over fifteen lengths and three nth positions with no mismatch.)"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "mimo-prismwing_amd", "csrc")


def test_register_nth_element_matches_libcxx_restatement(tmp_path):
    exe = str(tmp_path / "select_wave_check")
    subprocess.run(["g++", "-O2", "-std=c++20", "-pthread", "-I" + CSRC, os.path.join(HERE, "select_wave_check.cpp"),
                    "-o", exe], check=True, capture_output=True)
    out = subprocess.run([exe, "2", "quick"], capture_output=True, text=True, timeout=900)
    assert out.returncode == 0, out.stdout
    # five lengths x (three random patterns x 2 rows + five fixed patterns x 2 rows) x two nth positions,
    # then 4 expert counts x 7 whole routed rows, each checked by select_route_row and by fast_top8_set
    assert out.stdout.split() == ["rows", str(5 * 16 * 2 + 4 * 7 * 2), "mismatches", "0"], out.stdout
