"""HIP-graph replay timing, the method the reference tunes with (scripts/tune_table.py:38-57):
record a run of calls into a graph and time replays with events, so only GPU time counts.

Calls take a rotation index: the caller cycles through several copies of its weights so
that consecutive calls never find their operands in the 256 MB MALL or the L2.
"""
import statistics

import torch


def time_graph(call, rotations=1, calls_per_replay=20, replays=25):
    """Median microseconds per call over `replays` graph replays.

    call(i) issues one call using rotation i (0 <= i < rotations) on the current stream."""
    for i in range(rotations):
        call(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for r in range(calls_per_replay):
            call(r % rotations)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        graph.replay()
        en.record()
        en.synchronize()
        times.append(st.elapsed_time(en) * 1000.0 / calls_per_replay)
    del graph
    return statistics.median(times)


def rotations_for(bytes_per_copy, min_total=768 << 20, min_rot=2):
    """Copies needed so one full rotation streams at least `min_total` bytes."""
    return max(min_rot, -(-min_total // max(1, bytes_per_copy)))
