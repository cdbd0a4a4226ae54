"""Engine-side modules of the hot path: the audit plane, the audit kernel and the block-table view."""
