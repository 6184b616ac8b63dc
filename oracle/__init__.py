"""CPU oracle for the junqi_core rules: test infrastructure, never product code."""
