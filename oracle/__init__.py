"""TEST INFRASTRUCTURE ONLY -- CPU oracle for the mask-cost / assignment /
matched-loss path.  Importable only from tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package
(mask_loss_amd) never imports it."""
