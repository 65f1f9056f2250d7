"""Host logic of solarwm_amd/segments.py on the CPU: the teacher-forcing frame lists are the
oracle's key intervals (causal_model.py:434-468) expressed in frames; geometry errors."""

import pytest

from oracle import segments_ref as sr
from solarwm_amd.segments import teacher_forcing_frame_lists


def test_teacher_forcing_frame_lists_match_mask():
    """The product's frame lists are the oracle's key intervals, in frames."""
    for F, nb, sink, m in [(6, 2, 0, None), (6, 2, 2, 1), (9, 3, 3, 0), (8, 2, 4, 2)]:
        segs = sr.teacher_forcing_segments(num_frames=F, frame_seqlen=1, num_frame_per_block=nb,
                                           max_prior_clean_chunks=m, sink_size=sink)
        lists = teacher_forcing_frame_lists(num_frames=F, num_frame_per_block=nb,
                                            max_prior_clean_chunks=m, sink_size=sink)
        for (qs, qe, ivs), (f0, frames) in zip(segs, lists, strict=True):
            assert qs == f0 and sorted({t for a, b in ivs for t in range(a, b)}) == frames


def test_teacher_forcing_frame_list_errors():
    """The reference's checks and messages, in its order (causal_model.py:357-386)."""
    cases = [
        (dict(num_frames=6, num_frame_per_block=0), "num_frame_per_block must be positive, got 0"),
        (dict(num_frames=5, num_frame_per_block=2),
         "num_frames=5 must be divisible by num_frame_per_block=2"),
        (dict(num_frames=6, num_frame_per_block=2, sink_size=8), r"sink_size must be in \[0, 6\], got 8"),
        (dict(num_frames=6, num_frame_per_block=2, sink_size=-2), r"sink_size must be in \[0, 6\], got -2"),
        (dict(num_frames=6, num_frame_per_block=2, sink_size=1),
         "sink_size=1 must contain whole 2-frame chunks"),
        (dict(num_frames=6, num_frame_per_block=2, max_prior_clean_chunks=3),
         r"model.max_prior_clean_chunks must be in \[0, 2\] for a 3-chunk window, got 3"),
        (dict(num_frames=6, num_frame_per_block=2, max_prior_clean_chunks=-1),
         r"model.max_prior_clean_chunks must be in \[0, 2\] for a 3-chunk window, got -1"),
    ]
    for kw, msg in cases:
        with pytest.raises(ValueError, match="^" + msg + "$"):
            teacher_forcing_frame_lists(**kw)
