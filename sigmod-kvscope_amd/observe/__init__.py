"""Controller-side modules of the hot path: share normalisation, ranking, descriptor files."""
