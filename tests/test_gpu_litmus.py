"""Litmus for the grid barrier (grid_arrive / grid_wait) and the device-coherent
data path, through sinter_litmus_barrier (GPU).

Mirrors the reference's boundary litmus (tests/litmus_boundary.cu:1-18,
docs/SYNC-FINDINGS.md:9-32) for gfx950, where each of the 8 XCDs has its own
L2: every block publishes a payload word before arriving and, after the
crossing, reads the word of the next block -- dealt to another XCD -- whose
line it read (and so cached) before arriving; arrival order is shuffled by
pseudo-random delays every epoch.

Positive (the protocol the ops use: sc1 stores and loads, the flag barrier):
exactly-once counting (the final count is epochs * blocks, and no crossing
sees fewer than epoch * blocks arrivals) and no payload older than the epoch
over 100k epochs, with the reader's line pre-read plainly, coherently or not
at all.  Negatives break only the payload's visibility -- a plain cached
store, a plain cached load of a plainly pre-read line, a payload published
after arriving -- and each must be caught (stale reads observed) while the
barrier itself stays exact.  Measured on MI355X: a plain store is never seen
by another XCD during the run, a plain load of a plainly cached line stays
stale, a late publish is seen stale on ~12 % of the reads.  Every variant
waits only in the barrier's own bounded spin, so each kernel exits normally.
"""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu

BLOCKS = 256            # one workgroup per CU, the interpreter's grid


def _run(sn, mode, epochs, blocks=BLOCKS):
    counts = (C.c_uint64 * 3)()
    print(f"litmus mode {mode}: {blocks} blocks x {epochs} epochs", flush=True)
    sn.check(sn.lib().sinter_litmus_barrier(blocks, epochs, mode, counts), "litmus")
    stale, early, total = (int(v) for v in counts)
    print(f"litmus mode {mode}: stale {stale} early {early} arrivals {total}", flush=True)
    return stale, early, total


WARM_PLAIN, WARM_COHERENT = 0x10, 0x20


@pytest.mark.parametrize("warm", [0, WARM_PLAIN, WARM_COHERENT], ids=["no-preread", "plain-preread", "sc1-preread"])
def test_barrier_exactly_once_and_coherent_payload_fresh(sn, torch_gpu, warm):
    epochs = 100_000
    stale, early, total = _run(sn, 0 | warm, epochs)
    assert total == epochs * BLOCKS
    assert early == 0, "a crossing released before every arrival was counted"
    assert stale == 0, "a coherent payload read returned a previous epoch"


@pytest.mark.parametrize("mode,what", [(1, "plain store"), (2, "plain load of a pre-read line"),
                                       (3, "publish after arriving")])
def test_broken_payload_visibility_is_caught(sn, torch_gpu, mode, what):
    epochs = 20_000
    stale, early, total = _run(sn, mode | WARM_PLAIN, epochs)
    assert total == epochs * BLOCKS and early == 0   # the barrier itself is untouched
    assert stale > 0, f"the stale detector missed a {what}"


def test_litmus_refuses_bad_arguments(sn, torch_gpu):
    counts = (C.c_uint64 * 3)()
    L = sn.lib()
    assert L.sinter_litmus_barrier(1, 10, 0, counts) == sn.ERR_ARG       # a barrier needs two blocks
    assert L.sinter_litmus_barrier(BLOCKS, 10, 9, counts) == sn.ERR_ARG  # unknown mode
    assert L.sinter_litmus_barrier(BLOCKS, 10, 0x30, counts) == sn.ERR_ARG  # unknown pre-read
    assert L.sinter_litmus_barrier(BLOCKS, 0, 0, counts) == sn.ERR_ARG
