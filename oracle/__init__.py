"""CPU oracle for the AdaKV decode path (test infrastructure; never imported by adakv_amd)."""
