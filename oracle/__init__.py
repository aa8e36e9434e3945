"""CPU checker for race_attention_amd (test infrastructure only; never imported
by the product)."""
