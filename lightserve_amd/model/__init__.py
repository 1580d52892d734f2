"""LLaMA-shaped model around the MI355X attention (the reference's model/ package)."""
