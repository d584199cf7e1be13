"""``asc.lib``: the host-side runtime helpers of the reference (python/asc/lib/)."""
