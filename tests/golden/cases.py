"""Model settings of the golden cases (shared by make_golden.py and the tests)."""
SMALL = dict(n_basis=8, n_passes=2, radial_hidden=16, K_dir=4, norm="layer", transport=True, eqmsg=True,
             factor=True, B=8, K=16, rc=3.5)
FLAG = dict(n_basis=8, n_passes=2, radial_hidden=64, K_dir=16, norm="layer", transport=True, eqmsg=True,
            factor=True)

# name -> (model kwargs, elements, structure set); structure sets are built in make_golden.py
SMALL_CASES = {
    "small_flag_mol": (dict(SMALL, C=12), [1, 6, 8], "mols"),
    "small_flag_box": (dict(SMALL, C=12), [1, 6, 8], "box"),
    "small_cp_mol": (dict(SMALL, C=12, cp=True), [1, 6, 8], "mols"),
    "small_plain_box": (dict(SMALL, C=12, transport=False, eqmsg=False), [1, 6, 8], "box"),
    "small_3pass_mol": (dict(SMALL, C=8, n_passes=3), [1, 6, 8], "mols"),
}
BIG_CASES = {
    "cfg0_flag_c96": (dict(FLAG, C=96, B=16, K=32, rc=4.5), [1, 6, 8], "two"),
    "cfg1_cp_c160": (dict(FLAG, C=160, B=16, K=32, rc=4.5, cp=True), [1, 6, 8], "two"),
    "cfg2_flag_ag": (dict(FLAG, C=96, B=16, K=32, rc=4.5), [47], "fcc"),
    "cfg3_cp_c160": (dict(FLAG, C=160, B=16, K=32, rc=5.0, cp=True), [1, 6, 8], "liq"),
    "cfg4_flag_c256": (dict(FLAG, C=256, B=16, K=64, rc=5.5), [1, 6, 8], "liq"),
}
