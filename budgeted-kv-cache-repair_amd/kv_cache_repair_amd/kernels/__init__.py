"""MI355X (gfx950) HIP operators of the packed refresh executor."""
