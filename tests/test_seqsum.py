"""CPU proof of the exact parallel left-to-right binary32 sum
(gemma4.pas_amd/csrc/g4s_seqsum.h) that the full-vocabulary path uses for
LSum and for the draw's running sum (src/Gemma4.Tensors.pas:657-663,
src/Gemma4.Model.pas:2727-2735).  Every check compares against the literal
loop, bit for bit."""
import ctypes
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "native", "build", "libseqsum_check.so")


@pytest.fixture(scope="module")
def ss():
    if not os.path.exists(LIB):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
    L = ctypes.CDLL(LIB)
    L.ss_check_steps.restype = ctypes.c_int64
    L.ss_check_steps.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    L.ss_check_term_ct_f.restype = ctypes.c_int64
    L.ss_check_term_ct_f.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    L.ss_check_lane_map.restype = ctypes.c_int64
    L.ss_check_lane_map.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    L.ss_check_lane_map_fma.restype = ctypes.c_int64
    L.ss_check_lane_map_fma.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    L.ss_check_assoc.restype = ctypes.c_int64
    L.ss_check_assoc.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    L.ss_check_sequence.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_int64)]
    return L


def test_single_steps(ss):
    """RN32(S + a) from the term map, for S and a across every binade."""
    assert ss.ss_check_steps(1, 2_000_000) == 0


def test_float_term_classification_matches_integer(ss):
    """The binary32 form of a term's (c, t) used by the GPU kernels equals
    the integer form, for random terms including subnormals, in every
    binade near the term's own and in random binades."""
    assert ss.ss_check_term_ct_f(7, 300_000) == 0


def test_lane_map_matches_literal_loop(ss):
    """The single-pass lane map (parity chain with the first-tie offset)
    against the literal binary32 loop from even and odd entering sums, and
    against the composition of per-term maps."""
    assert ss.ss_check_lane_map(11, 400_000) == 0


def test_lane_map_fma_equals_lane_map(ss):
    """The one-pass form the bf16 map passes use for waves holding a tie
    (terms below 2^22 units; one tie in a lane closed-form, more take
    lane_map) gives lane_map's map exactly, from both parities."""
    assert ss.ss_check_lane_map_fma(12, 400_000) == 0


def test_composition_associative(ss):
    assert ss.ss_check_assoc(2, 200_000) == 0


KINDS = {0: "softmax terms", 1: "probabilities", 2: "8-bit mantissas (ties)",
         3: "powers of two and zeros", 4: "huge dynamic range", 5: "subnormals", 6: "uniform"}


@pytest.mark.parametrize("kind", sorted(KINDS))
@pytest.mark.parametrize("n,chunk,pt", [(1, 16, 4), (37, 16, 4), (5000, 1024, 16),
                                        (262144, 16384, 16)])
def test_sequences(ss, kind, n, chunk, pt):
    out = (ctypes.c_int64 * 5)()
    for seed in range(3 if n > 100000 else 12):
        for thr in (0.0, 0.3, 0.999, 1.0, 1.5):
            ss.ss_check_sequence(1000 * kind + seed, kind, n, chunk, pt, thr, out)
            assert out[0] == 0, (f"{KINDS[kind]} n={n} seed={seed} thr={thr}: "
                                 f"mismatch flags {out[0]} (accepted {out[1]}, re-evaluated "
                                 f"{out[2]}, rounds {out[3]})")


def test_long_row_mostly_accepts_chunk_maps(ss):
    """On a softmax-like row of 262144 terms, the chain accepts most chunk maps
    and re-evaluates only the few chunks where the sum changes binade."""
    out = (ctypes.c_int64 * 5)()
    ss.ss_check_sequence(7, 0, 262144, 16384, 16, 0.5, out)
    assert out[0] == 0
    assert out[1] >= 8 and out[2] <= 8, (out[1], out[2])
