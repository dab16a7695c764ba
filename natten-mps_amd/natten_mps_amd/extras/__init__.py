"""Extra operators outside the core neighbourhood-attention API
(``extras/`` of /root/reference/src/natten_mps)."""
