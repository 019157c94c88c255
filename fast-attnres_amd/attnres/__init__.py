"""Fast-AttnRes for AMD Instinct MI355X (gfx950).

Attention-Residuals reads ``attnres(values, query, *, eps, scale)`` computed
by hand-written HIP kernels behind a C ABI (`include/attnres_hip.h`), with
the public surface of the reference package: ``attnres``, ``LearnedQuery``
and ``__version__``.  ``SharedSources`` (no reference counterpart) runs
several reads of one source list with their source gradients summed in the
backward kernels.
"""

__version__ = "2.0.1+mi355x.1"

from .api import attnres
from .modules import LearnedQuery
from .shared import SharedSources, SourceBank

__all__ = ["LearnedQuery", "SharedSources", "SourceBank", "__version__", "attnres"]
