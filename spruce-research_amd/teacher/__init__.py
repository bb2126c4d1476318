"""Teacher target extraction (HIP): block attention mass and normalised targets."""
