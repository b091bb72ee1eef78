"""TEST INFRASTRUCTURE ONLY: CPU oracle for GGML_OP_FLASH_ATTN_EXT (see fa_oracle.c)."""
