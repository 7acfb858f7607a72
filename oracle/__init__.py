"""CPU oracle of the paged KV path — test infrastructure only (see kv_oracle.h)."""
