"""Writes tests/golden/mtx_golden.json: Matrix Market inputs and what the reference's reader and
COO -> CSR (include/mmio.hpp:19-75, include/csr.hpp:16-42) make of them -- the CSR arrays, or
the error text -- as printed by oracle/_ref/mtx_ref_dump (built by `make -C oracle ref` from the
reference's own headers).  Run in the build container, where the reference is present.

Each case is a file body; the fixture keeps the body and the reference's output."""
import json
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
DUMP = os.path.join(ROOT, "oracle", "_ref", "mtx_ref_dump")

B = "%%MatrixMarket matrix coordinate"
CASES = {
    # valid inputs
    "general_real": f"{B} real general\n% a comment\n\n3 4 5\n3 2 -1.5\n1 4 2e0\n1 1 0.25\n"
                    "2 3 +7\n3 4 1.e2\n",
    "general_crlf_tabs": f"{B} real general\r\n%c\r\n\r\n2 2 3\r\n2\t1\t-3.5E-2\r\n"
                         "1 2 .5\r\n  1   1   5.  \r\n",
    "symmetric_real": f"{B} real symmetric\n4 4 5\n1 1 2.0\n3 1 -1.0\n4 2 3.5\n4 4 1\n2 1 0.125\n",
    "skew_symmetric": f"{B} real skew-symmetric\n3 3 3\n2 1 1.5\n3 2 -2.25\n3 3 0\n",
    "pattern_general": f"{B} pattern general\n3 3 4\n1 3\n2 2\n3 1\n1 1\n",
    "pattern_symmetric": f"{B} pattern symmetric\n3 3 3\n2 1\n3 3\n3 2\n",
    "integer_general": f"{B} integer general\n2 3 3\n1 3 -4\n2 1 7\n1 1 0\n",
    "number_forms": f"{B} real general\n2 6 6\n1 1 007\n1 2 -0\n1 3 1e+2\n1 4 +1.5e-3\n"
                    "2 5 3.4028234e38\n2 6 1e-50\n",
    "comment_lines_between": f"{B} real general\n   % indented comment\n2 2 2\n%x\n"
                             "1 1 1\n \t\n2 2 2\n% trailing comment\n",
    "no_trailing_newline": f"{B} real general\n2 2 1\n2 2 9.5",
    "empty_rows_and_cols": f"{B} real general\n5 7 2\n5 7 1\n1 1 2\n",
    "zero_entries": f"{B} real general\n3 3 0\n",
    "unsorted_rows": f"{B} real general\n2 8 6\n2 8 1\n1 5 2\n2 1 3\n1 2 4\n2 4 5\n1 7 6\n",
    "dims_extra_tokens": f"{B} real general\n2 2 1 99\n1 1 1\n",
    # errors
    "empty_file": "",
    "bad_banner": "%%MatrixMarket matrix array real general\n2 2\n",
    "bad_magic": "%MatrixMarket matrix coordinate real general\n1 1 0\n",
    "complex_field": f"{B} complex general\n1 1 0\n",
    "hermitian": f"{B} real hermitian\n1 1 0\n",
    "missing_fields_banner": f"{B}\n1 1 0\n",
    "missing_dims": f"{B} real general\n% only comments\n",
    "bad_dims": f"{B} real general\n2 x 1\n",
    "dims_zero_rows": f"{B} real general\n0 2 0\n",
    "dims_count_too_big": f"{B} real general\n2 2 2147483648\n",
    "nonsquare_symmetric": f"{B} real symmetric\n2 3 0\n",
    "truncated": f"{B} real general\n2 2 3\n1 1 1\n2 2 2\n",
    "extra_entries": f"{B} real general\n2 2 1\n1 1 1\n2 2 2\n",
    "extra_field": f"{B} real general\n2 2 1\n1 1 1 5\n",
    "extra_field_pattern": f"{B} pattern general\n2 2 1\n1 1 1\n",
    "value_suffix": f"{B} real general\n2 2 1\n1 1 3.0x\n",
    "row_not_integer": f"{B} real general\n2 2 1\n1.5 1 3\n",
    "row_suffix": f"{B} real general\n2 2 1\n2x 1 3\n",
    "missing_value": f"{B} real general\n2 2 1\n1 1\n",
    "inf_token": f"{B} real general\n2 2 1\n1 1 inf\n",
    "nan_token": f"{B} real general\n2 2 1\n1 1 nan\n",
    "overflow_double": f"{B} real general\n2 2 1\n1 1 1e400\n",
    "beyond_float": f"{B} real general\n2 2 1\n1 1 1e39\n",
    "dangling_exponent": f"{B} real general\n2 2 1\n1 1 1e\n",
    "dot_exponent": f"{B} real general\n2 2 1\n1 1 .e5\n",
    "index_zero": f"{B} real general\n2 2 1\n0 1 1\n",
    "index_past_end": f"{B} real general\n2 2 1\n1 3 1\n",
    "index_overflow": f"{B} real general\n2 2 1\n99999999999999999999 1 1\n",
    "skew_diagonal": f"{B} real skew-symmetric\n2 2 1\n2 2 1.0\n",
    "duplicate": f"{B} real general\n2 2 2\n1 2 1\n1 2 3\n",
    "duplicate_by_symmetry": f"{B} real symmetric\n2 2 2\n2 1 1\n1 2 3\n",
}


def main():
    if not os.path.exists(DUMP):
        sys.exit(f"{DUMP} is not built (make -C oracle ref)")
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name, body in CASES.items():
            path = os.path.join(tmp, name + ".mtx")
            with open(path, "w", newline="") as fh:
                fh.write(body)
            r = subprocess.run([DUMP, path], capture_output=True, text=True, check=True)
            out[name] = {"body": body, "reference": r.stdout}
    with open(os.path.join(HERE, "mtx_golden.json"), "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
    print(f"{len(out)} cases")


if __name__ == "__main__":
    main()
