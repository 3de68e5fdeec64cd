"""CPU oracle for the KVM forward path (test infrastructure only)."""
