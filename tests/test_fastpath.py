"""CPU checks of the fast projections (coset_amd/csrc/e8_fast.hpp): the
encoder's project_fast, the decoders' project_dyadic and their short
residual residual_dyadic (with a negative control that must fail).

The header is compiled for the host (tests/fastpath/Makefile) and checked
against the C oracle's projection: exhaustively for the rounding lemma it
rests on (every float below 2^22), with a looser tie limit as the negative
control that must fail, and bit for bit on blocks from eight input families
(Gaussian at eight scales, dyadic grids, near-ties, points on the boundary
between the two D8 cosets, specials, uniform, tiny and sparse blocks)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(__file__), "fastpath")
EXE = os.path.join(HERE, "_build", "check_fastpath")
# the library headers the mutated copies do not replace (fastdiv.hpp)
CSRC = os.path.join(HERE, "..", "..", "coset_amd", "csrc")


@pytest.fixture(scope="module")
def checker():
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    subprocess.run(["make", "-s", "-C", HERE], check=True, capture_output=True)
    return EXE


def run(exe, *args):
    p = subprocess.run([exe, *args], capture_output=True, text=True, timeout=600)
    return p.returncode, p.stdout


def test_rounding_lemma_exhaustive(checker):
    rc, out = run(checker, "lemma")
    assert rc == 0, out
    assert " 0 inexact" in out and " 0 custom_round != rint" in out, out


def test_rounding_lemma_fails_at_the_tie(checker):
    """Negative control: at |t - rint t| < 1/2 the lemma is false, so the
    exhaustive check must report the floats where custom_round differs."""
    rc, out = run(checker, "lemma", "0.5")
    assert rc == 1, out


def test_fast_projection_matches_oracle(checker):
    """Both forms of the fast path: the strict one (conditions (1)-(4)) and
    the generic encoder's, which also takes blocks that condition (5)
    decides for the D8 candidate (tiny blocks, exact zeros)."""
    rc, out = run(checker, "blocks", "300000", "11")
    assert rc == 0, out
    lines = [l for l in out.splitlines() if l.startswith("family")]
    rates = {int(l.split()[1].rstrip(":")): float(l.split("(")[1].split("%")[0]) for l in lines}
    rates5 = {int(l.split()[1].rstrip(":")): float(l.split("(")[3].split("%")[0]) for l in lines}
    assert len(rates) == 8
    assert rates[6] > 99.0, out   # uniform box: almost always fast
    assert rates[4] > 10.0, out   # near coset boundaries: many decided, the rest fall back
    assert all(rates5[f] >= rates[f] for f in rates), out
    assert rates[7] < 20.0 and rates5[7] > 90.0, out   # tiny and sparse blocks: (5) decides them


def test_condition5_fails_without_its_d8_term(tmp_path):
    """Negative control of condition (5): with the D8 candidate's adjustment
    term dropped (2 - sum |d0_i| > 2^-14 alone), the bound no longer holds
    and the checker must find blocks whose rows differ from the oracle's.
    The mutated header is a copy built here; the library's is untouched."""
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    src = os.path.join(HERE, "..", "..", "coset_amd", "csrc", "e8_fast.hpp")
    text = open(src).read()
    term = "(decided || base - t0 > kFastDistGap)"
    assert text.count(term) == 1, "condition (5) moved: update this negative control"
    inc = tmp_path / "inc"
    inc.mkdir()
    (inc / "e8_fast.hpp").write_text(text.replace(term, "(decided || base > kFastDistGap)"))
    for name in os.listdir(os.path.dirname(src)):
        if name.endswith(".hpp") and name != "e8_fast.hpp":
            shutil.copy(os.path.join(os.path.dirname(src), name), inc / name)
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    oracle = os.path.join(HERE, "..", "..", "oracle", "e8_oracle.c")
    exe = tmp_path / "check_mutated"
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=c99", "-ffp-contract=off", "-fno-fast-math", "-c", "-o",
                    str(tmp_path / "o.o"), oracle], check=True, capture_output=True)
    subprocess.run([hipcc, "-O2", "-std=c++17", "-ffp-contract=off", "--offload-arch=gfx950", f"-I{inc}", f"-I{CSRC}", "-c",
                    "-o", str(tmp_path / "c.o"), os.path.join(HERE, "check_fastpath.hip")], check=True,
                   capture_output=True)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-o", str(exe), str(tmp_path / "c.o"), str(tmp_path / "o.o"),
                    "-lpthread", "-lm"], check=True, capture_output=True)
    rc, out = run(str(exe), "blocks", "300000", "11")
    assert rc == 1, out
    bad = [l for l in out.splitlines() if l.startswith("family") and not l.endswith("row mismatches 0")]
    assert len(bad) >= 3, out   # several families hit blocks where the dropped term matters


@pytest.mark.parametrize("q,n", [(2, 1 << 20), (4, 1 << 20), (8, 1 << 24), (16, 1000000)])
def test_dyadic_projection_matches_oracle(checker, q, n):
    """The decoders' exact projection of G b / q for q = 2^k: every code for
    q <= 8 (16.7 M at q = 8), a structured and random sample at q = 16,
    residuals equal to the oracle's under both distance rules."""
    rc, out = run(checker, "dyadic", str(q), str(n))
    assert rc == 0, out
    assert " mismatches 0" in out, out


@pytest.mark.parametrize("q,n", [(8, 1 << 24), (16, 1 << 21), (32, 1 << 20)])
def test_fast_residual_matches_oracle(checker, q, n):
    """The decoders' short residual residual_dyadic<q> (straight from the
    digits, |d1| = 1/2 - |d0|, b - a = 2 - sum |d0| + corrections): every
    code at q = 8, the structured codes and a random sample at q = 16 and
    32, bit for bit against the oracle's residual under both distance rules.
    (Every one of the 2^32 codes at q = 16 is checked by
    `check_fastpath fastres 16 4294967296 <threads>`, about ten minutes on
    eight cores.)"""
    rc, out = run(checker, "fastres", str(q), str(n), str(min(8, os.cpu_count() or 1)))
    assert rc == 0, out
    assert " mismatches 0" in out, out


@pytest.mark.parametrize("q,n", [(2, 1 << 8), (4, 1 << 16), (8, 1 << 24), (16, 1 << 21)])
def test_table_residual_matches_oracle(checker, q, n):
    """The integer decode dyadic_level_acc<q> of the layer round-trip kernel
    and the QAT backward (per-coordinate table, first-index argmax/argmin as
    maxima of packed keys, sums and parities as one add): every code at
    q = 2, 4 and 8, the structured codes and a random sample at q = 16,
    twice the residual bit for bit against the oracle's under both distance
    rules.  (All 2^32 codes at q = 16:
    `check_fastpath tabres 16 4294967296 <threads>`, about ten minutes on
    eight cores.)"""
    rc, out = run(checker, "tabres", str(q), str(n), str(min(8, os.cpu_count() or 1)))
    assert rc == 0, out
    assert " mismatches 0" in out, out


def test_table_residual_fails_with_a_wrong_gx_direction(tmp_path):
    """Negative control of the table decode: with the D8 + 1/2 candidate's g_x
    direction taken from the sign of d1 alone (without z >= 1/2), the
    checker must report mismatches.  The mutated header is a copy built
    here."""
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    src = os.path.join(HERE, "..", "..", "coset_amd", "csrc", "e8_fast.hpp")
    text = open(src).read()
    term = "c1 = Z >= Q && d1 > 0;"
    assert text.count(term) == 1, "the table's c1 rule moved: update this negative control"
    inc = tmp_path / "inc"
    inc.mkdir()
    (inc / "e8_fast.hpp").write_text(text.replace(term, "c1 = d1 > 0;"))
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    oracle = os.path.join(HERE, "..", "..", "oracle", "e8_oracle.c")
    exe = tmp_path / "check_mutated"
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=c99", "-ffp-contract=off", "-fno-fast-math", "-c", "-o",
                    str(tmp_path / "o.o"), oracle], check=True, capture_output=True)
    subprocess.run([hipcc, "-O2", "-std=c++17", "-ffp-contract=off", "--offload-arch=gfx950", f"-I{inc}", f"-I{CSRC}",
                    "-c", "-o", str(tmp_path / "c.o"), os.path.join(HERE, "check_fastpath.hip")], check=True,
                   capture_output=True)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-o", str(exe), str(tmp_path / "c.o"), str(tmp_path / "o.o"),
                    "-lpthread", "-lm"], check=True, capture_output=True)
    rc, out = run(str(exe), "tabres", "8", str(1 << 24), "4")
    assert rc == 1, out
    assert " mismatches 0" not in out, out


def test_fast_residual_fails_without_its_integer_tie_rule(tmp_path):
    """Negative control of residual_dyadic: without the nudge that sends the
    D8 + 1/2 candidate of a positive integer z to z - 1 (custom_round's tie
    toward zero at z - 1/2), the checker must report mismatches.  The
    mutated header is a copy built here; the library's is untouched."""
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    src = os.path.join(HERE, "..", "..", "coset_amd", "csrc", "e8_fast.hpp")
    text = open(src).read()
    term = "constexpr float kNudge = 1.f / (float)(4 * Q);"
    assert text.count(term) == 1, "residual_dyadic's nudge moved: update this negative control"
    inc = tmp_path / "inc"
    inc.mkdir()
    (inc / "e8_fast.hpp").write_text(text.replace(term, "constexpr float kNudge = 0.f;"))
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    oracle = os.path.join(HERE, "..", "..", "oracle", "e8_oracle.c")
    exe = tmp_path / "check_mutated"
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=c99", "-ffp-contract=off", "-fno-fast-math", "-c", "-o",
                    str(tmp_path / "o.o"), oracle], check=True, capture_output=True)
    subprocess.run([hipcc, "-O2", "-std=c++17", "-ffp-contract=off", "--offload-arch=gfx950", f"-I{inc}", f"-I{CSRC}", "-c",
                    "-o", str(tmp_path / "c.o"), os.path.join(HERE, "check_fastpath.hip")], check=True,
                   capture_output=True)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-o", str(exe), str(tmp_path / "c.o"), str(tmp_path / "o.o"),
                    "-lpthread", "-lm"], check=True, capture_output=True)
    rc, out = run(str(exe), "fastres", "8", str(1 << 24), "4")
    assert rc == 1, out
    assert " mismatches 0" not in out, out


@pytest.mark.parametrize("steps,k", [(1, 256), (2, 256)])
def test_division_by_reciprocal(checker, steps, k):
    """div_by_recip (the layer round trip's dec / beta from one reciprocal per
    block) against the IEEE quotient: every significand of b in [1, 2) with
    a = 0, 1/2, .., 128 (and the four sign pairs on every 16th b), plus, with
    two corrections, random a and b over the helper's whole exponent domain.
    (The single correction's range that the kernel relies on, every
    half-integer up to 16384, is checked by `check_fastpath divq 1 32768
    <threads>`, about six minutes on eight cores.)"""
    rc, out = run(checker, "divq", str(steps), str(k), str(min(8, os.cpu_count() or 1)))
    assert rc == 0, out
    assert " mismatches 0" in out, out


def test_division_by_reciprocal_fails_without_its_correction(checker):
    """Negative control: the bare product RN(a RN(1/b)) is not the correctly
    rounded quotient, so the checker must find mismatches without the
    correction step."""
    rc, out = run(checker, "divq", "0", "16", str(min(8, os.cpu_count() or 1)))
    assert rc == 1, out
    assert " mismatches 0" not in out, out


def test_row_index_by_multiplier(checker):
    """u32div (the layer round trip's row of a block, floor(i / blocks_per_row)
    from a host-computed multiplier) against integer division: every divisor
    below 2^16, powers of two and their neighbours, 2^32 - 1 and random
    divisors, at the numerators next to their multiples, the range's ends and
    random ones."""
    rc, out = run(checker, "u32div", "100000")
    assert rc == 0, out
    assert " mismatches 0" in out, out
