"""The traffic summary's source hash (bench.kernel_source_sha256) follows the
decode kernel's code, not its comments or layout."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_comments_and_layout_are_ignored():
    a = 'int f(int x) {  // twice x\n  return 2 * x; /* a\n block */ }\n'
    b = '/* header */\nint f(int x) {\n\n    return 2 * x;   }  // end\n'
    assert bench.code_without_comments(a) == bench.code_without_comments(b)
    assert bench.code_without_comments(a) == "int f(int x) { return 2 * x; }"


def test_code_changes_are_seen():
    a = "int f(int x) { return 2 * x; }"
    assert bench.code_without_comments(a) != bench.code_without_comments(a.replace("2", "3"))
    # a token split by blank space is not a token joined
    assert bench.code_without_comments("a b") != bench.code_without_comments("ab")


def test_literals_are_kept_whole():
    src = 'const char* s = "a // not a comment /* nor this */";  char c = \'"\'; // gone\n'
    assert bench.code_without_comments(src) == (
        'const char* s = "a // not a comment /* nor this */"; char c = \'"\';')
    esc = 'p("quote \\" // still inside"); // out'
    assert bench.code_without_comments(esc) == 'p("quote \\" // still inside");'


def test_committed_summary_matches_these_sources():
    traffic, source, note = bench.measured_traffic("c2")
    assert traffic is not None, note
    assert source == os.path.join("profiles", "paged_decode_write_kernel_c2_traffic.md")
