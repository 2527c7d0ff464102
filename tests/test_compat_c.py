"""The drop-in claim from C: a C11 caller that uses qw6's Vulkan host-op
names (qw6_vk.h:9-56), built with the reference's own warning flags
(-std=c11 -Wall -Wextra -Werror -Wpedantic, the reference Makefile:5)
against include/qw6_hip_compat.h, links against libqw6_hip.so and gets
qw6's -1 on every argument the library rejects before device work (no GPU
needed)."""
import subprocess
from pathlib import Path

import qw6_amd as Q

ROOT = Path(__file__).resolve().parents[1]

CALLER = r"""
#include <stdio.h>
#include <stdint.h>
#include "qw6_hip_compat.h"

static int fails = 0;
#define EXPECT_FAIL(call) do { if ((call) != -1) { fprintf(stderr, "accepted: %s\n", #call); fails++; } } while (0)

int main(void) {
    float x[512] = {0}, y[512] = {0}, w[512] = {0}, val = 0.0f;
    uint32_t idx[8] = {0}, tok = 0;
    unsigned char q[2048] = {0};
    int (*selftest)(void) = qw6_vk_selftest;   /* linked, not run: it needs a GPU */

    EXPECT_FAIL(qw6_vk_matvec_f32_host(NULL, x, y, 4, 4));
    EXPECT_FAIL(qw6_vk_matvec_f32_host(w, x, y, 0, 4));
    EXPECT_FAIL(qw6_vk_matmul_q4k_host(q, x, y, 1, 100));         /* cols % 256 */
    EXPECT_FAIL(qw6_vk_matmul_q5k_host(NULL, x, y, 1, 256));
    EXPECT_FAIL(qw6_vk_matmul_q6k_host(q, x, NULL, 1, 256));
    EXPECT_FAIL(qw6_vk_matmul_iq2xxs_host(q, x, y, 1, 300));
    EXPECT_FAIL(qw6_vk_rmsnorm_host(x, w, y, 0, 1e-6f));
    EXPECT_FAIL(qw6_vk_silu_mul_host(x, NULL, y, 4));
    EXPECT_FAIL(qw6_vk_argmax_host(x, 0, idx, &val));
    EXPECT_FAIL(qw6_vk_argmax_host(NULL, 4, idx, &val));
    EXPECT_FAIL(qw6_vk_sampling_greedy_host(x, 0, &tok));
    EXPECT_FAIL(qw6_vk_moe_route_host(x, idx, w, 300, 8));        /* n_experts > 256 */
    EXPECT_FAIL(qw6_vk_moe_route_host(x, idx, w, 16, 9));         /* top_k > 8 */
    EXPECT_FAIL(qw6_vk_moe_gather_host(x, w, NULL, 0.0f, y, 4, 9));
    if (!selftest) fails++;
    if (qw6_hip_last_error()[0] == '\0') fails++;                 /* the message of the last rejection */
    printf("%s %d\n", fails ? "FAIL" : "ok", fails);
    return fails != 0;
}
"""


def test_c11_caller_of_vk_names_links_and_gets_minus_one(tmp_path):
    src = tmp_path / "caller.c"
    src.write_text(CALLER)
    exe = tmp_path / "caller"
    lib_dir = Q.LIB_PATH.parent
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wpedantic", "-O2",
           "-I" + str(ROOT / "include"), "-o", str(exe), str(src),
           "-L" + str(lib_dir), "-l:" + Q.LIB_PATH.name, "-Wl,-rpath," + str(lib_dir),
           "-Wl,-rpath,/opt/rocm/lib", "-Wl,--allow-shlib-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok 0", (r.stdout, r.stderr)
