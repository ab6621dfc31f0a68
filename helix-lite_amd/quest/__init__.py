"""Quest decode-time page selection (drop-in for the reference's ``quest``
package, src/quest/__init__.py:22-34), on gfx950 kernels."""
from .reference import (  # noqa: F401
    compute_page_stats,
    page_upper_bound,
    selected_attention,
    topk_pages_with_sinks,
)

__all__ = [
    "compute_page_stats",
    "page_upper_bound",
    "topk_pages_with_sinks",
    "selected_attention",
]
