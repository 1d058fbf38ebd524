"""volta_amd -- MI355X (gfx950) drop-in for Volta's compile-train MLP step."""
