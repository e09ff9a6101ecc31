"""Developer tools around the mi355x target (per-tensor debug dumps)."""
