"""The hand-over the one-launch decode step rests on, measured through htr_debug_handover (csrc/handover.hip): a word
stored at workgroup scope is seen by an agent-scope load of a workgroup on the same XCD — the premise of the step's
two XCD-local hand-overs (workgroups 0 and 8 share an XCD: a launch spreads its workgroups round-robin over the 8, as
the step's own placement check confirms) — one stored at agent scope is seen from another XCD, and all-to-all
exchanges of 256 … 3072 words complete. The arguments the probe refuses."""
import pytest

import htr

pytestmark = pytest.mark.gpu


def test_workgroup_scope_word_is_seen_on_its_xcd(dev):
    us, seen = dev.handover(0, 0, 8, iters=500)
    print(f"\n[hand-over] workgroup-scope word, one XCD: {us:.3f} µs a round trip", flush=True)
    assert seen and 0 < us < 100


def test_agent_scope_word_is_seen_across_xcds(dev):
    us, seen = dev.handover(1, 0, 1, iters=500)
    print(f"\n[hand-over] agent-scope word, two XCDs: {us:.3f} µs a round trip", flush=True)
    assert seen and 0 < us < 100


@pytest.mark.parametrize("words", [256, 1024, 3072])
def test_all_to_all_exchange_completes(dev, words):
    us, seen = dev.handover(2, words=words, iters=100)
    print(f"\n[hand-over] all-to-all of {words} words: {us:.3f} µs an exchange", flush=True)
    assert seen and 0 < us < 1000


def test_handover_arguments_refused(dev):
    with pytest.raises(htr.HtrError, match="two of 0"):
        dev.handover(0, 3, 3)
    with pytest.raises(htr.HtrError, match="multiple of 256"):
        dev.handover(2, words=1000)
    with pytest.raises(htr.HtrError, match="kind 3"):
        dev.handover(3)
