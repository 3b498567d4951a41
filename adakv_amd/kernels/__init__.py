"""HIP kernel entry points for gfx950 (MI355X)."""
