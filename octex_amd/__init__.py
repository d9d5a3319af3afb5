"""octex for MI355X: approximate k-nearest-neighbor search by E8-lattice cell lists (cuvs::neighbors::octex),
with every search step a hand-written HIP kernel for gfx950.

    import octex_amd as octex
    index = octex.load("index_dir")        # or octex.build(xb, "index_dir")
    D, I = index.search(xq, k=10)          # (distances, neighbors), nearest first

Drop-ins: `from octex_amd import cuvs as cagra` (cuvs.neighbors.cagra calls) and `from octex_amd import faiss`
(Faiss GPU index calls).
"""

from .index import Index, build, build_in_memory, load

__version__ = "0.1.0"
__all__ = ["Index", "build", "build_in_memory", "load", "__version__"]
