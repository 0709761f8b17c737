"""The message-graph cache evicts entries (it is cleared once it holds more than eight graphs),
while a captured HIP graph keeps using the raw addresses of the CSR tensors it recorded.
``pin_graphs`` must keep every graph handed out inside its scope alive after eviction.
CPU only: the CSR build is plain torch and runs on CPU tensors."""
import gc
import weakref

import torch

from ictc_o3.backends.hip import graph_message as gm


def _edges(seed, nodes=7, edges=20):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(0, nodes, (edges,), generator=g),
            torch.randint(0, nodes, (edges,), generator=g))


def test_pinned_graphs_survive_cache_eviction():
    src, dst = _edges(0)
    with gm.pin_graphs() as held:
        graph = gm.message_graph(src, dst, 7, 7)
        again = gm.message_graph(src, dst, 7, 7)          # cache hit: pinned once
    assert again is graph and len(held) == 1 and held[0] is graph
    refs = [weakref.ref(t) for t in (graph.rowptr_dst, graph.perm_dst, graph.rowptr_src, graph.perm_src)
            if t is not None]
    assert refs
    del graph, again
    for seed in range(1, 12):                             # cycle the cache past its clearing point
        gm.message_graph(*_edges(seed), 7, 7)
    gm._GRAPH_CACHE.clear()
    gc.collect()
    assert all(r() is not None for r in refs)
    held.clear()
    gc.collect()
    assert all(r() is None for r in refs)


def test_unpinned_scope_collects_nothing():
    with gm.pin_graphs() as outer:
        with gm.pin_graphs() as inner:
            g1 = gm.message_graph(*_edges(20), 7, 7)
        g2 = gm.message_graph(*_edges(21), 7, 7)
    assert inner == [g1] and outer == [g1, g2]
    gm.message_graph(*_edges(22), 7, 7)                   # outside every scope
    assert outer == [g1, g2] and not gm._PIN_LISTS
