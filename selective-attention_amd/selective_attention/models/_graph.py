"""Greedy decoding with the decode step captured in a HIP graph."""
from __future__ import annotations

import torch


def graph_decode(body, calls: int, on_token, done, check_every: int = 16) -> int:
    """Run `body` (one decode step that reads and rewrites its own static
    tensors: the token, the caches, the lengths) `calls` times: the first call
    eagerly on a side stream (which also warms the libraries' per-stream
    state), the rest as replays of its graph, captured on that stream.
    on_token(i) runs after call i (1-based); done() is polled every
    `check_every` calls and stops the loop when true.  Returns the number of
    calls made."""
    if calls <= 0 or done():
        return 0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    on_token(1)
    if calls == 1:
        return 1
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        body()
    made = 1
    while made < calls:
        if made % check_every == 0 and done():
            break
        graph.replay()
        made += 1
        on_token(made)
    return made
