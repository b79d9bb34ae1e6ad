"""Model-level examples built on the ConvRot linear."""
