"""Cache of superoptimize results (python/yirage/graph_dataset.py of the
reference): entries are keyed by the input graph's owner-independent hash
and matched on every search argument plus the backend."""
from __future__ import annotations


class DatasetEntry:
    def __init__(self, input_graph, optimized_graph, imaps, omaps, griddims, blockdims, fmaps, franges, backend):
        self.input_graph = input_graph
        self.optimized_graph = optimized_graph
        self.key = (imaps, omaps, griddims, blockdims, fmaps, franges, backend)


class GraphDataset:
    def __init__(self):
        self.dataset: dict = {}

    def find(self, input_graph, imaps, omaps, griddims, blockdims, fmaps, franges, backend):
        key = (imaps, omaps, griddims, blockdims, fmaps, franges, backend)
        for e in self.dataset.get(input_graph.get_owner_independent_hash(), []):
            if e.key == key:
                return e.optimized_graph
        return None

    def store(self, input_graph, optimized_graph, imaps, omaps, griddims, blockdims, fmaps, franges, backend):
        e = DatasetEntry(input_graph, optimized_graph, imaps, omaps, griddims, blockdims, fmaps, franges, backend)
        self.dataset.setdefault(input_graph.get_owner_independent_hash(), []).append(e)

    def clear(self):
        self.dataset.clear()


graph_dataset = GraphDataset()
