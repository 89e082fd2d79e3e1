"""Structure input (include/hkbs_structure.h) on the CPU.

Pinned three ways: known answers the mathematics fixes (template geometry,
virtual-CB coefficients, a rigid fit recovering a known motion), the
behaviour the reference's own loader tests assert (tests/cpp/
structure_input_tests.cpp, residue_template_frozen_tests.cpp), and field-by-
field equality with the reference's loader compiled into oracle/_ref on the
parity fixtures, on randomised PDB / mmCIF scenes and on every error path.
"""
from __future__ import annotations

import numpy as np
import pytest

from hikoboshi_amd import backbone
from hikoboshi_amd import structure as S
from hikoboshi_amd.exceptions import HikoboshiError, InvalidArgumentError, UnavailableError

from .conftest import FIXTURES

CODES = {"invalid_argument": 1, "failed_precondition": 2, "unavailable": 3, "unimplemented": 4, "internal_error": 5}
THREE = ["ALA", "ARG", "ASN", "ASP", "CYS", "GLN", "GLU", "GLY", "HIS", "ILE", "LEU", "LYS", "MET", "PHE", "PRO",
         "SER", "THR", "TRP", "TYR", "VAL"]
ATOMS = ["N", "CA", "C", "O", "CB"]
MISSING, OBSERVED, INFERRED, VIRTUAL = 0, 1, 2, 3


# ------------------------------------------------------------ rendering ----
def pdb_atom(serial, name, resn, chain, num, xyz, *, het=False, altloc=" ", icode=" ", occ=1.0):
    """One fixed-column ATOM/HETATM record (PDB format v3.3 columns)."""
    label = name if len(name) == 4 else f" {name:<3}"
    rec = "HETATM" if het else "ATOM  "
    return (f"{rec}{serial:5d} {label}{altloc}{resn:>3} {chain or ' '}{num:4d}{icode}   "
            f"{xyz[0]:8.3f}{xyz[1]:8.3f}{xyz[2]:8.3f}{occ:6.2f}{0.0:6.2f}          {name[0]:>2}")


def to_pdb(models, *, crlf=False, wrap_models=True):
    """models: list of (model number, records); records are dicts of pdb_atom's fields."""
    lines = []
    serial = 1
    for num, recs in models:
        if wrap_models:
            lines.append(f"MODEL     {num:4d}")
        for r in recs:
            lines.append(pdb_atom(serial, r["name"], r["resn"], r["chain"], r["num"], r["xyz"], het=r["het"],
                                  altloc=r["alt"], icode=r["icode"]))
            serial += 1
        lines.append("TER")
        if wrap_models:
            lines.append("ENDMDL")
    lines.append("END")
    return ("\r\n" if crlf else "\n").join(lines) + "\n"


CIF_COLUMNS = ["group_PDB", "id", "type_symbol", "label_atom_id", "label_alt_id", "label_comp_id", "label_asym_id",
               "auth_asym_id", "label_seq_id", "auth_seq_id", "pdbx_PDB_ins_code", "Cartn_x", "Cartn_y", "Cartn_z",
               "occupancy", "auth_comp_id", "auth_atom_id", "pdbx_PDB_model_num"]


def to_mmcif(models, rng, *, drop=(), model_tokens=None):
    """The same records as an mmCIF _atom_site loop with shuffled columns, some quoted tokens, '.'/'?' for
    blanks, some rows wrapped over two lines and a preceding non-atom_site loop."""
    cols = [c for c in CIF_COLUMNS if c not in drop]
    rng.shuffle(cols)
    out = ["data_synthetic", "#", "loop_", "_entity_poly.entity_id", "_entity_poly.type", "1 'polypeptide(L)'", "#",
           "loop_"] + [f"_atom_site.{c}" for c in cols]
    serial = 1
    for num, recs in models:
        for r in recs:
            v = {
                "group_PDB": "HETATM" if r["het"] else "ATOM", "id": str(serial), "type_symbol": r["name"][0],
                "label_atom_id": r["name"], "auth_atom_id": r["name"],
                "label_alt_id": "." if r["alt"] == " " else r["alt"], "label_comp_id": r["resn"],
                "auth_comp_id": r["resn"], "label_asym_id": r["chain"] or ".", "auth_asym_id": r["chain"] or "?",
                "label_seq_id": str(r["num"]), "auth_seq_id": str(r["num"]),
                "pdbx_PDB_ins_code": "?" if r["icode"] == " " else r["icode"],
                "Cartn_x": f"{r['xyz'][0]:.3f}", "Cartn_y": f"{r['xyz'][1]:.3f}", "Cartn_z": f"{r['xyz'][2]:.3f}",
                "occupancy": "1.00", "pdbx_PDB_model_num": (model_tokens or {}).get(num, str(num)),
            }
            toks = []
            for c in cols:
                t = v[c]
                q = rng.random()
                toks.append(f'"{t}"' if q < 0.1 else f"'{t}'" if q < 0.2 else t)
            if rng.random() < 0.1:
                k = int(rng.integers(1, len(toks)))
                out += [" ".join(toks[:k]), "  " + " ".join(toks[k:])]
            else:
                out.append(" ".join(toks))
            serial += 1
    out += ["#", "loop_", "_pdbx_struct_oper_list.id", "1", "#"]
    return "\n".join(out) + "\n"


def records_from_pdb(text, chain=None, drop_every=0):
    """Records of a PDB file's ATOM lines (optionally relabelled to one chain and thinned: O and CB removed
    from every drop_every-th residue; a template fit on the remaining N, CA, C restores them, whereas a
    fit that includes a real O or CB exceeds the 0.5 A guard)."""
    recs = []
    for ln in (ln for ln in text.splitlines() if ln.startswith("ATOM")):
        name = ln[12:16].strip()
        if drop_every and name in ("O", "CB") and int(ln[22:26]) % drop_every == 0:
            continue
        recs.append(dict(name=name, resn=ln[17:20].strip(), chain=chain or ln[21].strip(), num=int(ln[22:26]),
                         xyz=(float(ln[30:38]), float(ln[38:46]), float(ln[46:54])), het=False, alt=ln[16],
                         icode=ln[26]))
    return recs


def scene(seed, *, n_models=1):
    """A randomised structure: a water chain, two polymer chains (B before A) with modified, unknown and
    HETATM-canonical residues, side-chain atoms, dropped and distorted atoms, altlocs, insertion codes and
    numbering gaps; optional extra models with shifted coordinates."""
    rng = np.random.default_rng(seed)
    models = []
    chain_len = {"B": int(rng.integers(3, 9)), "A": int(rng.integers(4, 12))}
    base = {c: backbone.single_chain(n, seed * 7 + i).coords for i, (c, n) in enumerate(chain_len.items())}
    plan = {}
    for c, n in chain_len.items():
        res = []
        num = int(rng.integers(-3, 20))
        for i in range(n):
            kind = rng.random()
            resn = THREE[int(rng.integers(0, 20))]
            het = False
            if kind < 0.08:
                resn, het = ["MSE", "SEP", "HYP", "TPO"][int(rng.integers(0, 4))], True
            elif kind < 0.12:
                resn = "UNK"
            elif kind < 0.15:
                het = True  # a canonical name on HETATM records is not a polymer residue
            elif kind < 0.25:
                resn = "GLY"
            step = 1 if rng.random() < 0.85 else int(rng.integers(2, 5))
            icode = " "
            if rng.random() < 0.1 and i > 0:
                step, icode = 0, "AB"[int(rng.integers(0, 2))]
            num += step
            drop = {a for a in ATOMS if rng.random() < 0.12}
            if rng.random() < 0.05:
                drop |= {"N", "CA", "C"} - {ATOMS[int(rng.integers(0, 3))]}
            distort = rng.random() < 0.1
            alts = rng.random() < 0.15
            res.append(dict(i=i, resn=resn, het=het, num=num, icode=icode, drop=drop, distort=distort, alts=alts))
        plan[c] = res
    for m in range(n_models):
        recs = []
        if m == 0 or rng.random() < 0.5:
            recs.append(dict(name="O", resn="HOH", chain="W", num=1, xyz=(50.0, 50.0, 50.0), het=True, alt=" ",
                             icode=" "))
        for c, res in plan.items():
            xyz_all = base[c] + 30.0 * m + (0.0 if c == "A" else 15.0)
            for r in res:
                names = ATOMS[:4] + ([] if r["resn"] == "GLY" else ["CB"]) + ["CG", "OXT"]
                for a in names:
                    if a in r["drop"]:
                        continue
                    k = ATOMS.index(a) if a in ATOMS else 4
                    xyz = xyz_all[r["i"], k] + (1.5 if a in ("CG", "OXT") else 0.0)
                    if r["distort"] and a in ("O", "C"):
                        xyz = xyz + rng.normal(0, 1.2, 3)
                    rec = dict(name=a, resn=r["resn"], chain=c, num=r["num"], xyz=xyz, het=r["het"], alt=" ",
                               icode=r["icode"])
                    if r["alts"] and a in ATOMS and rng.random() < 0.6:
                        order = rng.permutation(["A", "B", " ", "a", "C"])[: int(rng.integers(2, 4))]
                        for alt in order:
                            recs.append(dict(rec, alt=alt, xyz=xyz + rng.normal(0, 0.3, 3)))
                    else:
                        recs.append(rec)
        recs.append(dict(name="FE", resn="HEM", chain="A", num=900, xyz=(1.0, 2.0, 3.0), het=True, alt=" ",
                         icode=" "))
        models.append((m + 1, recs))
    return models


# ----------------------------------------------------------- comparison ----
def ours(*, path=None, content=None, fmt="pdb", label="", model_index=None, model_id="", chain_id="",
         chain_index=None, infer=True, include_modified=True):
    opts = S.StructureLoadOptions(model_index=model_index, model_id=model_id, chain_id=chain_id,
                                  chain_index=chain_index, infer_missing_atoms=infer,
                                  include_modified_residues=include_modified)
    try:
        if path is not None:
            st = S.load_structure_from_file(path, opts)
        elif fmt == "pdb":
            st = S.load_pdb_from_string(content, label, opts)
        else:
            st = S.load_mmcif_from_string(content, label, opts)
    except HikoboshiError as exc:
        return CODES[exc.code], exc.detail, None
    return 0, "", st


def assert_same(reference, **kw):
    st_r, msg_r, r = reference.load_structure(**kw)
    st_o, msg_o, o = ours(**kw)
    assert (st_o, msg_o) == (st_r, msg_r)
    if r is None:
        return None
    assert o.coords.view(np.uint32).tobytes() == r["coords"].view(np.uint32).tobytes()
    np.testing.assert_array_equal(o.atom_sources, r["atom_sources"])
    assert o.residue_codes == r["residue_codes"]
    np.testing.assert_array_equal(o.numbering["residue_numbers"], r["residue_numbers"])
    np.testing.assert_array_equal(o.numbering["insertion_codes"], r["insertion_codes"])
    np.testing.assert_array_equal(o.numbering["source_record_indices"], r["source_record_indices"])
    assert o.chain_breaks == r["chain_breaks"]
    assert [m.original_residue_name for m in o.residues] == r["residue_names"]
    assert (o.input_id, o.source_filename, o.selected_model_id, o.selected_chain_id, o.altloc_note,
            o.selected_model_index) == (r["input_id"], r["source_filename"], r["model_id"], r["chain_id"],
                                        r["altloc_note"], r["model_index"])
    return o


# ------------------------------------------------------ known answers ----
def test_template_geometry_is_the_frozen_one():
    """An ALA whose N, CA, C sit exactly on the residue template receives the template's O and CB (a rigid
    fit of the template onto itself is the identity); values frozen by residue_template_frozen_tests.cpp."""
    tmpl_n, tmpl_ca, tmpl_c = (-1.458, 0.0, 0.0), (0.0, 0.0, 0.0), (1.4213556, 0.5526060, 0.0)
    text = "\n".join(pdb_atom(i + 1, a, "ALA", "A", 1, xyz) for i, (a, xyz) in
                     enumerate(zip(["N", "CA", "C"], [tmpl_n, tmpl_ca, tmpl_c])))
    st = S.load_pdb_from_string(text, "t.pdb")
    assert list(st.atom_sources[0]) == [OBSERVED, OBSERVED, OBSERVED, INFERRED, INFERRED]
    np.testing.assert_allclose(st.coords[0, 3], (1.6192990, 1.7675873, 0.0), atol=1e-3)
    np.testing.assert_allclose(st.coords[0, 4], (0.0596943, -0.2987801, -0.4695088), atol=1e-3)
    # the template's bond lengths
    assert np.linalg.norm(st.coords[0, 3] - st.coords[0, 2]) == pytest.approx(1.231, abs=2e-3)


def test_virtual_cb_coefficients():
    """Glycine CB from N=(0,0,0), CA=(1,0,0), C=(1,1,0): CA + a*(b x c) + b'*b + c'*c with the ProteinMPNN
    coefficients gives (1.5680283, -0.5406747, -0.5827343)."""
    text = "\n".join(pdb_atom(i + 1, a, "GLY", "A", 1, xyz) for i, (a, xyz) in
                     enumerate(zip(["N", "CA", "C"], [(0, 0, 0), (1, 0, 0), (1, 1, 0)])))
    st = S.load_pdb_from_string(text, "g.pdb")
    assert st.atom_sources[0, 4] == VIRTUAL
    np.testing.assert_allclose(st.coords[0, 4], (1.5680283, -0.5406747, -0.5827343), atol=2e-6)
    np.testing.assert_array_equal(st.coords[0, 4], backbone.virtual_cb(*[st.coords[0, k] for k in range(3)]))


@pytest.mark.parametrize("seed", range(6))
def test_rigid_fit_recovers_a_known_motion(seed):
    """Missing atoms of a rigidly moved template come back at the moved template positions."""
    rng = np.random.default_rng(seed)
    q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    q *= np.sign(np.linalg.det(q))
    shift = rng.normal(0, 20, 3)
    tmpl = np.array([(-1.458, 0, 0), (0, 0, 0), (1.4213556, 0.5526060, 0), (1.6192990, 1.7675873, 0),
                     (0.0596943, -0.2987801, -0.4695088)])
    moved = tmpl @ q.T + shift
    keep = [0, 1, 2, 3, 4]
    gone = sorted(rng.choice(5, size=int(rng.integers(1, 3)), replace=False))
    text = "\n".join(pdb_atom(i + 1, ATOMS[k], "SER", "A", 1, moved[k]) for i, k in enumerate(keep) if k not in gone)
    st = S.load_pdb_from_string(text, "m.pdb")
    for k in gone:
        assert st.atom_sources[0, k] == INFERRED
        np.testing.assert_allclose(st.coords[0, k], moved[k], atol=3e-3)  # input rounded to 1e-3 A


def test_inference_guards():
    """Fewer than three anchors, collinear anchors or a fit worse than 0.5 A leave atoms Missing."""
    two = "\n".join(pdb_atom(i + 1, a, "ALA", "A", 1, xyz) for i, (a, xyz) in
                    enumerate(zip(["N", "CA"], [(0, 0, 0), (1.458, 0, 0)])))
    st = S.load_pdb_from_string(two, "two.pdb")
    assert list(st.atom_sources[0]) == [OBSERVED, OBSERVED, MISSING, MISSING, MISSING]
    assert not st.coords[0, 2:].any()
    line = "\n".join(pdb_atom(i + 1, a, "ALA", "A", 1, (1.5 * i, 0, 0)) for i, a in enumerate(["N", "CA", "C"]))
    assert list(S.load_pdb_from_string(line, "l.pdb").atom_sources[0]) == [1, 1, 1, 0, 0]
    bad = "\n".join(pdb_atom(i + 1, a, "ALA", "A", 1, xyz) for i, (a, xyz) in
                    enumerate(zip(["N", "CA", "C", "O"], [(0, 0, 0), (1.458, 0, 0), (2.9, 0.55, 0), (9, 9, 9)])))
    assert S.load_pdb_from_string(bad, "b.pdb").atom_sources[0, 4] == MISSING
    off = S.load_pdb_from_string(bad.replace("(9", "(3"), "b.pdb",
                                 S.StructureLoadOptions(infer_missing_atoms=False))
    assert off.atom_sources[0, 4] == MISSING


def test_glycine_without_backbone_keeps_cb_missing():
    text = "\n".join(pdb_atom(i + 1, a, "GLY", "A", 1, xyz) for i, (a, xyz) in
                     enumerate(zip(["CA", "C"], [(1, 0, 0), (1, 1, 0)])))
    st = S.load_pdb_from_string(text, "g.pdb")
    assert st.atom_sources[0, 4] == MISSING and st.atom_sources[0, 3] == MISSING
    # computed from N = origin all the same, as ProteinMPNN's _get_cb does
    np.testing.assert_array_equal(st.coords[0, 4], backbone.virtual_cb(np.zeros(3), st.coords[0, 1], st.coords[0, 2]))


def _residue(chain, num, resn="ALA", origin=(0.0, 0.0, 0.0), het=False, alt=" ", atoms=ATOMS, serial=1):
    o = np.asarray(origin, float)
    geo = [(0, 0, 0), (1.458, 0, 0), (2.0, 1.42, 0), (3.2, 1.5, 0.3), (1.9, -0.8, 1.2)]
    return [pdb_atom(serial + i, a, resn, chain, num, o + geo[ATOMS.index(a)], het=het, altloc=alt)
            for i, a in enumerate(atoms)]


def test_selection_behaviour_of_the_reference_tests():
    """The behaviours tests/cpp/structure_input_tests.cpp asserts, on inputs of our own."""
    two_chains = "\n".join(_residue("B", 1, "VAL", (30, 0, 0)) + _residue("A", 1) + _residue("A", 2, "GLY", (4, 0, 0)))
    st = S.load_pdb_from_string(two_chains, "x.pdb")
    assert st.selected_chain_id == "A" and st.residue_codes == "AG"
    assert S.load_pdb_from_string(two_chains, "x.pdb", S.StructureLoadOptions(chain_index=0)).residue_codes == "V"
    water_first = "\n".join([pdb_atom(1, "O", "HOH", "W", 1, (50, 50, 50), het=True)] + _residue("B", 1, "VAL"))
    st = S.load_pdb_from_string(water_first, "w.pdb")
    assert st.selected_chain_id == "B" and st.residue_count == 1
    models = "\n".join(["MODEL        1"] + _residue("A", 1) + ["ENDMDL", "MODEL        2"] +
                       _residue("A", 1, origin=(100, 0, 0)) + ["ENDMDL"])
    assert S.load_pdb_from_string(models, "m.pdb").coords[0, 0, 0] == 0.0
    m2 = S.load_pdb_from_string(models, "m.pdb", S.StructureLoadOptions(model_index=2))
    assert m2.coords[0, 0, 0] == 100.0 and m2.selected_model_id == "2"
    alt = "\n".join(_residue("A", 1, alt="A") + _residue("A", 1, origin=(999, 99, 0), alt="B", atoms=["N", "CA"]))
    st = S.load_pdb_from_string(alt, "alt.pdb")
    assert st.residue_count == 1 and st.coords[0, 0, 0] == 0.0
    per_atom = "\n".join(_residue("A", 1, atoms=["N"]) + _residue("A", 1, origin=(100, 0, 0), alt="A", atoms=["CA"]) +
                         _residue("A", 1, atoms=["CA", "C", "O", "CB"]))
    st = S.load_pdb_from_string(per_atom, "pa.pdb")
    assert st.coords[0, 1, 0] == pytest.approx(1.458) and st.altloc_note == "altloc selection applied"
    mse = "\n".join(_residue("A", 1, "MSE", het=True) + [pdb_atom(9, "O", "HOH", "A", 100, (50, 50, 50), het=True)])
    st = S.load_pdb_from_string(mse, "mse.pdb")
    assert st.residue_codes == "M" and st.residues[0].original_residue_name == "MSE"
    gap = "\n".join(_residue("A", 1) + _residue("A", 2, origin=(4, 0, 0)) + _residue("A", 5, origin=(12, 0, 0)))
    assert S.load_pdb_from_string(gap, "gap.pdb").chain_breaks == (1,)


def test_invalid_coordinates_are_rejected():
    good = pdb_atom(1, "N", "ALA", "A", 1, (11.104, 13.207, 10.0))
    for bad in (good[:30] + "  XX.XXX" + good[38:], good[:30] + "     nan" + good[38:], good[:30] + "     inf" + good[38:]):
        with pytest.raises(InvalidArgumentError, match="invalid coordinate field; refusing to silently zero-fill"):
            S.load_pdb_from_string(bad, "bad.pdb")
    with pytest.raises(UnavailableError, match="structure file not readable"):
        S.load_structure_from_file("/nonexistent/x.pdb")


def test_format_detection():
    assert S.detect_structure_format("a.PDB", "") == "pdb" and S.detect_structure_format("a.Ent", "") == "pdb"
    assert S.detect_structure_format("a.cif", "") == "mmcif" and S.detect_structure_format("a.MMCIF", "") == "mmcif"
    assert S.detect_structure_format("", "data_x\n") == "mmcif"
    assert S.detect_structure_format("", "HEADER\n_atom_site.id\n") == "mmcif"
    assert S.detect_structure_format("", "REMARK\nMODEL        1\n") == "pdb"
    assert S.detect_structure_format("a.txt", "random text") == "unknown"


# ------------------------------------------------- reference comparison ----
@pytest.mark.parametrize("name", sorted(p.name for p in FIXTURES.glob("*.pdb")))
def test_fixtures_match_reference_loader(reference, name):
    o = assert_same(reference, path=str(FIXTURES / name))
    assert o.residue_count > 0 and (o.atom_sources > 0).all()
    for kw in (dict(chain_index=0), dict(chain_id="A"), dict(model_id="1"), dict(infer=False), dict(chain_id="Q"),
               dict(chain_index=3), dict(model_index=2)):
        assert_same(reference, path=str(FIXTURES / name), **kw)


def test_fixtures_mutilated_match_reference_loader(reference, tmp_path):
    """Real geometry with atoms removed and displaced, so every inference branch runs on real residues."""
    rng = np.random.default_rng(5)
    for name in sorted(p.name for p in FIXTURES.glob("*.pdb")):
        lines = (FIXTURES / name).read_text().splitlines()
        out = []
        for ln in lines:
            if ln.startswith("ATOM") and ln[12:16].strip() in ATOMS:
                u = rng.random()
                if u < 0.15:
                    continue
                if u < 0.2:
                    x = float(ln[30:38]) + rng.normal(0, 0.8)
                    ln = ln[:30] + f"{x:8.3f}" + ln[38:]
            out.append(ln)
        p = tmp_path / name
        p.write_text("\n".join(out) + "\n")
        o = assert_same(reference, path=str(p))
        assert (o.atom_sources == INFERRED).any()


SCENE_OPTIONS = [dict(), dict(chain_id="B"), dict(chain_index=1), dict(chain_index=2), dict(model_index=2),
                 dict(model_id="2"), dict(infer=False), dict(include_modified=False), dict(chain_id="W"),
                 dict(chain_id="Z"), dict(model_index=5), dict(model_id="x")]


@pytest.mark.parametrize("seed", range(24))
def test_pdb_scenes_match_reference_loader(reference, seed):
    models = scene(seed, n_models=1 + seed % 3)
    text = to_pdb(models, crlf=seed % 5 == 4, wrap_models=seed % 3 != 0)
    for kw in SCENE_OPTIONS:
        assert_same(reference, content=text, fmt="pdb", label=f"scene{seed}.pdb", **kw)


@pytest.mark.parametrize("seed", range(24))
def test_mmcif_scenes_match_reference_loader(reference, seed):
    rng = np.random.default_rng(1000 + seed)
    models = scene(seed, n_models=1 + seed % 3)
    drops = [(), ("auth_asym_id",), ("auth_seq_id", "auth_comp_id"), ("label_atom_id",), ("label_alt_id",
             "pdbx_PDB_ins_code", "pdbx_PDB_model_num", "group_PDB")][seed % 5]
    tokens = {2: "02"} if seed % 4 == 1 else None
    text = to_mmcif(models, rng, drop=drops, model_tokens=tokens)
    for kw in SCENE_OPTIONS + [dict(model_id="02")]:
        assert_same(reference, content=text, fmt="mmcif", label=f"scene{seed}.cif", **kw)


def test_files_and_format_dispatch_match_reference(reference, tmp_path):
    rng = np.random.default_rng(3)
    models = scene(3, n_models=2)
    pdb_text, cif_text = to_pdb(models), to_mmcif(models, rng)
    cases = {"a.pdb": pdb_text, "b.ENT": pdb_text, "c.cif": cif_text, "d.mmCIF": cif_text, "e.txt": pdb_text,
             "f": cif_text, "g.dat": "nothing to see\n", "h.pdb": cif_text, "i.cif": pdb_text, "j.pdb": ""}
    for fname, text in cases.items():
        p = tmp_path / fname
        p.write_text(text)
        assert S.detect_structure_format(str(p), text) == reference.detect_structure_format(str(p), text)
        assert_same(reference, path=str(p))
    assert_same(reference, path=str(tmp_path / "missing.pdb"))
    assert_same(reference, path=str(tmp_path))  # a directory reads as empty


def _bad(line, start, width, text):
    return line[:start] + text.rjust(width)[:width] + line[start + width:]


def pdb_error_cases():
    base = pdb_atom(1, "N", "ALA", "A", 1, (1.0, 2.0, 3.0))
    ca = pdb_atom(2, "CA", "ALA", "A", 1, (2.0, 2.0, 3.0))
    return {
        "short record": base[:53],
        "serial": _bad(base, 6, 5, "x1"),
        "plus serial": _bad(base, 6, 5, "+12"),
        "residue number": _bad(base, 22, 4, "1a"),
        "negative number": _bad(base, 22, 4, "-7"),
        "coordinate garbage": _bad(base, 30, 8, "1.0x"),
        "coordinate hex": _bad(base, 30, 8, "0x1p3"),
        "coordinate exponent": _bad(base, 30, 8, "1e2"),
        "coordinate plus minus": _bad(base, 30, 8, "+-1.5"),
        "coordinate inf": _bad(base, 38, 8, "inf"),
        "coordinate empty": _bad(base, 46, 8, ""),
        "model serial": "MODEL     x\n" + base,
        "no records": "HEADER    nothing\nEND\n",
        "empty": "",
        "only water": pdb_atom(1, "O", "HOH", "A", 1, (0, 0, 0), het=True),
        "only ligand atoms": pdb_atom(1, "FE", "HEM", "A", 1, (0, 0, 0), het=True),
        "unknown residue": base + "\n" + pdb_atom(2, "CA", "XYZ", "A", 2, (0, 0, 0)),
        "lower altloc": base + "\n" + _bad(ca, 16, 1, "a") + "\n" + _bad(ca, 16, 1, "B"),
        "blank chain": _bad(base, 21, 1, " ") + "\n" + _bad(ca, 21, 1, " "),
        "tab padded": base.replace("  1.000", "\t 1.000"),
        "model outside": base + "\nMODEL        2\n" + ca + "\nENDMDL\n" + ca,
    }


@pytest.mark.parametrize("case", sorted(pdb_error_cases()))
def test_pdb_edge_cases_match_reference_loader(reference, case):
    text = pdb_error_cases()[case]
    for kw in (dict(), dict(model_index=2), dict(chain_id="A")):
        assert_same(reference, content=text, fmt="pdb", label="e.pdb", **kw)


def cif_error_cases():
    head = ["data_x", "loop_", "_atom_site.group_PDB", "_atom_site.label_atom_id", "_atom_site.auth_comp_id",
            "_atom_site.auth_asym_id", "_atom_site.auth_seq_id", "_atom_site.Cartn_x", "_atom_site.Cartn_y",
            "_atom_site.Cartn_z"]
    row = "ATOM CA ALA A 1 1.0 2.0 3.0"
    return {
        "no loop": "data_x\n_cell.length_a 10\n",
        "no rows": "\n".join(head + ["#"]) + "\n",
        "no atom name": "\n".join(h for h in head if "atom_id" not in h) + "\nATOM ALA A 1 1.0 2.0 3.0\n",
        "no z": "\n".join(head[:-1]) + "\nATOM CA ALA A 1 1.0 2.0\n",
        "short row": "\n".join(head + ["ATOM CA ALA A 1 1.0 2.0"]),
        "wrapped row": "\n".join(head + ["ATOM CA ALA", "A 1 1.0", "2.0 3.0", "#"]),
        "bad number": "\n".join(head + ["ATOM CA ALA A 1x 1.0 2.0 3.0"]),
        "dot number": "\n".join(head + ["ATOM CA ALA A . 1.0 2.0 3.0"]),
        "bad coordinate": "\n".join(head + ["ATOM CA ALA A 1 1.0abc 2.0 3.0"]),
        "unknown coordinate": "\n".join(head + ["ATOM CA ALA A 1 ? 2.0 3.0"]),
        "quoted": "\n".join(head + ['ATOM "CA" \'ALA\' A 1 1.0 2.0 3.0', "ATOM 'C'x ALA A 1 2.0 2.0 3.0"]),
        "empty quoted": "\n".join(head + ['ATOM CA ALA "" 1 1.0 2.0 3.0']),
        "extra tokens": "\n".join(head + [row + " extra tokens", "#"]),
        "two blocks": "\n".join(head + [row, "#"] + head + ["ATOM N ALA A 1 0.0 2.0 3.0"]),
        "repeated column": "\n".join(head + ["_atom_site.auth_seq_id", row + " 7"]),
        "blank lines": "\n".join(head[:4] + ["", "   "] + head[4:] + ["", row, "", "ATOM N ALA A 1 0 0 0"]) + "\n\n",
        "other category inside": "\n".join(head + ["_other.x"] + [row]),
        "crlf": "\r\n".join(head + [row, "#"]) + "\r\n",
        "model token": "\n".join(head + ["_atom_site.pdbx_PDB_model_num", row + " 01", row.replace("1.0", "9.0") + " x"]),
    }


@pytest.mark.parametrize("case", sorted(cif_error_cases()))
def test_mmcif_edge_cases_match_reference_loader(reference, case):
    text = cif_error_cases()[case]
    for kw in (dict(), dict(model_id="01"), dict(model_index=1), dict(chain_id="A")):
        assert_same(reference, content=text, fmt="mmcif", label="e.cif", **kw)


@pytest.mark.parametrize("seed", range(8))
def test_pdb_fuzz_matches_reference_loader(reference, seed):
    """Random byte changes inside the fixed columns of a scene's records."""
    rng = np.random.default_rng(seed)
    lines = to_pdb(scene(100 + seed, n_models=2)).splitlines()
    alphabet = list(" 0123456789.-+eEABxn\t")
    for _ in range(25):
        mutated = list(lines)
        for _ in range(int(rng.integers(1, 4))):
            k = int(rng.integers(0, len(mutated)))
            ln = list(mutated[k])
            if ln:
                j = int(rng.integers(0, len(ln)))
                ln[j] = alphabet[int(rng.integers(0, len(alphabet)))]
            mutated[k] = "".join(ln)
        assert_same(reference, content="\n".join(mutated) + "\n", fmt="pdb", label="fuzz.pdb")


# ------------------------------------------------ Python entry points ----
def test_inverse_fold_selection_keywords(tmp_path):
    """Selection keywords of hikoboshi.inverse_fold (python/hikoboshi/_chain_resolve.py,
    cpp/include/hikoboshi/bindings/engine_helpers.hpp:302-332) reach the loader; errors before any design."""
    import warnings

    from hikoboshi_amd import inverse_fold as ifold
    from hikoboshi_amd.exceptions import InternalError

    fix = sorted(FIXTURES.glob("*.pdb"))
    recs = records_from_pdb(fix[0].read_text(), "A") + records_from_pdb(fix[1].read_text(), "B", drop_every=4)
    path = tmp_path / "two.cif"
    path.write_text(to_mmcif([(1, recs)], np.random.default_rng(0)))
    bb, native = ifold.load_structure(str(path))
    assert bb.L == len(S.load_structure_from_file(fix[0]).residue_codes)
    bb_b, native_b = ifold.load_structure(str(path), chain_id="B")
    assert native_b == S.load_structure_from_file(fix[1]).residue_codes
    assert (bb_b.atom_sources == INFERRED).any()
    assert ifold.load_structure(str(path), chain_index=1)[1] == native_b
    with pytest.raises(InvalidArgumentError, match="requested chain id not present in selected model"):
        ifold.load_structure(str(path), chain_id="C")
    with pytest.raises(InvalidArgumentError, match="selected model index not present in input"):
        ifold.load_structure(str(path), pdb_model_index=2)
    with pytest.raises(InvalidArgumentError, match="requested model id not present in input"):
        ifold.load_structure(str(path), pdb_model_id="7")
    f = ifold.inverse_fold
    with pytest.raises(InvalidArgumentError, match="choose either chain_id or chain_index, not both"):
        f.from_cif(str(path), chain_id="A", chain_index=0)
    with pytest.raises(InvalidArgumentError, match="choose either pdb_model_id or pdb_model_index, not both"):
        f(str(path), pdb_model_id="1", pdb_model_index=1)
    with pytest.raises(InvalidArgumentError, match="unknown inverse_fold.from_structure keyword[(]s[)]: bogus, zz"):
        f(str(path), zz=1, bogus=2)
    with pytest.raises(InvalidArgumentError, match="chain_index must be an int"):
        f(str(path), chain_index="1")
    with pytest.raises(InternalError, match="can't convert negative int to unsigned"):
        f(str(path), chain_index=-1)
    with pytest.raises(InvalidArgumentError, match="choose either pdb_model_id or deprecated model_id"):
        f(str(path), model_id="1", pdb_model_id="1")
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        with pytest.raises(InvalidArgumentError, match="requested chain id not present"):
            f(str(path), model_index=1, chain_id="Z")
    assert any("model_index is deprecated; use pdb_model_index" in str(w.message) for w in caught)
    # decode order is checked before the structure is read, the package after
    with pytest.raises(InvalidArgumentError, match="decode_order must be"):
        f(str(tmp_path / "missing.pdb"), decode_order="c_to_n")
    with pytest.raises(UnavailableError, match="structure file not readable"):
        f(str(tmp_path / "missing.pdb"), package="nope")
    opts = ifold.structure_options(pdb_model_index=2**32 + 2, chain_index=3)
    assert opts.model_index == 2 and opts.chain_index == 3
    # several chains (extension): labels and offsets reach the backbone
    bb2, native2 = ifold.load_structure(str(path), all_chains=True)
    assert native2 == native + native_b and bb2.L == bb.L + bb_b.L
    np.testing.assert_array_equal(bb2.chain_labels, np.repeat([0, 1], [bb.L, bb_b.L]))
    assert ifold.load_structure(str(path), chain_ids=["B", "A"])[1] == native_b + native
    with pytest.raises(InvalidArgumentError, match="choose one chain selection"):
        f(str(path), chain_ids=["A"], chain_id="A")
    with pytest.raises(InvalidArgumentError, match="chain_ids must be a sequence of chain id strings"):
        f(str(path), chain_ids="AB")


# ---------------------------------------------------- several chains ----
def _block_equals_single_chain(multi, single, rows):
    assert multi.coords[rows].view(np.uint32).tobytes() == single.coords.view(np.uint32).tobytes()
    np.testing.assert_array_equal(multi.atom_sources[rows], single.atom_sources)
    assert "".join(multi.residue_codes[i] for i in rows) == single.residue_codes
    for key in ("residue_numbers", "insertion_codes", "source_record_indices"):
        np.testing.assert_array_equal(multi.numbering[key][rows], single.numbering[key])
    assert [multi.residues[i].original_residue_name for i in rows] == [m.original_residue_name for m in single.residues]


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("fmt", ["pdb", "mmcif"])
def test_several_chains_are_single_chain_loads_side_by_side(seed, fmt):
    """all_chains / chain_ids (an extension of the reference's one-chain selection): each chain's block is
    exactly that chain's own load; chain breaks are the per-chain breaks shifted to the block; labels index
    the selected chains."""
    models = scene(seed, n_models=1 + seed % 2)
    text = to_pdb(models) if fmt == "pdb" else to_mmcif(models, np.random.default_rng(seed))
    load = S.load_pdb_from_string if fmt == "pdb" else S.load_mmcif_from_string
    for opts in (S.StructureLoadOptions(all_chains=True), S.StructureLoadOptions(chain_ids=("A", "B")),
                 S.StructureLoadOptions(chain_ids=("B", "A"), model_index=1 + seed % 2, infer_missing_atoms=seed % 3 > 0)):
        multi = load(text, "m", opts)
        expect = ("B", "A") if opts.all_chains else opts.chain_ids
        assert multi.chain_ids == expect and multi.selected_chain_id == ",".join(expect)
        labels = multi.chain_labels
        assert (np.diff(labels) >= 0).all() and set(labels) == set(range(len(expect)))
        breaks = []
        for c, cid in enumerate(expect):
            single = load(text, "m", S.StructureLoadOptions(chain_id=cid, model_index=opts.model_index,
                                                           infer_missing_atoms=opts.infer_missing_atoms))
            rows = np.flatnonzero(labels == c)
            assert rows.size == single.residue_count
            _block_equals_single_chain(multi, single, rows)
            assert all(multi.residues[i].chain_id == cid for i in rows)
            breaks += [int(rows[0]) + b for b in single.chain_breaks]
        assert multi.chain_breaks == tuple(breaks)
        bb = multi.backbone()
        np.testing.assert_array_equal(bb.chain_labels, labels)
        np.testing.assert_array_equal(bb.residue_indices, np.arange(multi.residue_count) + 100 * labels)
    one = load(text, "m")
    assert one.chain_ids == ("A",) and not one.chain_labels.any() and one.backbone().residue_indices is None


def test_several_chains_errors():
    text = to_pdb(scene(2))
    cases = [(dict(chain_ids=("A", "Q")), "requested chain id not present in selected model"),
             (dict(chain_ids=("A", "A")), "chain ids must be distinct"),
             (dict(chain_ids=("A",), chain_id="B"), "choose one chain selection"),
             (dict(all_chains=True, chain_index=0), "choose one chain selection"),
             (dict(all_chains=True, chain_ids=("A",)), "choose one chain selection"),
             (dict(chain_ids=()), "chain_ids must name at least one chain")]
    for kw, msg in cases:
        with pytest.raises(InvalidArgumentError, match=msg):
            S.load_pdb_from_string(text, "e", S.StructureLoadOptions(**kw))
    # the reference's own precedence stays: chain_id over chain_index
    assert S.load_pdb_from_string(text, "e", S.StructureLoadOptions(chain_id="B", chain_index=0)).chain_ids == ("B",)
    water = pdb_atom(1, "O", "HOH", "W", 1, (0, 0, 0), het=True) + "\n" + "\n".join(_residue("B", 1, "VAL"))
    assert S.load_pdb_from_string(water, "w", S.StructureLoadOptions(all_chains=True)).chain_ids == ("B",)
    with pytest.raises(InvalidArgumentError, match="selected model has no polymer chains"):
        S.load_pdb_from_string(pdb_atom(1, "O", "HOH", "W", 1, (0, 0, 0), het=True), "w",
                               S.StructureLoadOptions(all_chains=True))
