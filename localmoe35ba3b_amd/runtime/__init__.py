"""Runtime layer: route plans, routed MoE and the HBM-resident synthetic stack."""
