"""Item dealing of the prefill grouped GEMM (item_deal.h, dynamic_items in
grouped_gemm.hip): every (M tile, N tile) item is drawn exactly once over
the XCDs' counters, the shared expert's M tiles by N blocks per XCD, first,
M tiles fastest, and every other M tile whole by the XCD that owns it.
Checked by brute force in a host build of the header (tests/item_deal) over
the shapes the library launches (T = 4096 at d = 6144: 256 routed tiles + 22
shared; gate/up 8 N tiles of 512 weight rows, down 16 of 384) and over random
shapes, and with no shared group (the
dealing before it: whole M tiles round-robin)."""
import os
import random
import subprocess

DRIVER_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "item_deal")


def run_cases(cases):
    subprocess.run(["make", "-s", "-C", DRIVER_DIR], check=True)
    text = "".join(f"{m} {p} {x} {sm}\n" for m, p, x, sm in cases)
    r = subprocess.run([os.path.join(DRIVER_DIR, "driver")], input=text, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == f"ok {len(cases)}"


def test_dealing_of_the_benchmark_shapes():
    # prefill T = 4096: 256 routed M tiles + 22 shared (192 rows), 8 N tiles
    # for gate/up (256 h columns) and 16 for down (384 columns); on the
    # 160-row list, 256 + 26 M tiles and 8 N tiles for gate/up (256 h
    # columns), 12 for down (512 columns: blocks of 1 and 2 N tiles); a Zipf
    # batch with multi-tile hot experts; no shared expert.
    run_cases([(278, 8, 8, 22), (278, 16, 8, 22), (282, 8, 8, 26), (282, 12, 8, 26),
               (300, 8, 8, 22), (300, 16, 8, 22), (310, 8, 8, 26), (310, 12, 8, 26),
               (256, 16, 8, 0), (9, 16, 8, 1)])


def test_dealing_of_random_shapes():
    rng = random.Random(7)
    cases = []
    for _ in range(400):
        nxcd = rng.choice([1, 2, 4, 8])
        per_m = rng.choice([nxcd * rng.randint(1, 6), rng.randint(1, 50)])
        m_tiles = rng.randint(nxcd, 400)
        sh_m = rng.choice([0, rng.randint(1, min(m_tiles, 40))])
        cases.append((m_tiles, per_m, nxcd, sh_m))
    run_cases(cases)
