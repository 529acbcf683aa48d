"""ArcLight flash attention on MI355X (gfx950)."""
