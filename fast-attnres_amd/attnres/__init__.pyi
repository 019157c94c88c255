from torch import Tensor

from .modules import LearnedQuery as LearnedQuery
from .shared import SharedSources as SharedSources
from .shared import SourceBank as SourceBank

__version__: str


def attnres(
    values: Tensor | list[Tensor] | tuple[Tensor, ...],
    query: Tensor,
    *,
    eps: float = ...,
    scale: float = ...,
) -> Tensor: ...


__all__ = ["LearnedQuery", "SharedSources", "SourceBank", "__version__", "attnres"]
