/* Host test of include/bonsai_p40_dispatch.h: the cases of the reference's
 * test_dispatch_predicate (tests/test_p40.cpp:653-698), plain C. */
#include <stdio.h>
#include "../../include/bonsai_p40_dispatch.h"

static int fails = 0, passes = 0;
#define CHECK(c, msg) do { if (c) ++passes; else { ++fails; printf("FAIL: %s\n", msg); } } while (0)

static bonsai_mulmat_shape base(void) {
    bonsai_mulmat_shape s = {BONSAI_GGML_TYPE_PQ2_0, BONSAI_GGML_TYPE_F32, BONSAI_GGML_TYPE_F32,
                             5120, 17408, 1, 1, 1, 1, 1, 1, (5120 / 128) * 34};
    return s;
}

int main(void) {
    bonsai_mulmat_shape s = base();
    CHECK(bonsai_decode_path_ok(&s), "accepts ffn_up 5120 -> 17408");
    const long long widths[] = {5120, 17408, 6144, 10240, 12288, 1024};
    for (int i = 0; i < 6; ++i) {
        s = base(); s.n_in = widths[i]; s.nb1 = widths[i] / 128 * 34;
        CHECK(bonsai_decode_path_ok(&s), "accepts a model width");
    }
    s = base(); s.type0 = 1;  CHECK(!bonsai_decode_path_ok(&s), "rejects F16 weights");
    s = base(); s.type0 = 42; CHECK(!bonsai_decode_path_ok(&s), "rejects Q2_0 (42)");
    s = base(); s.type1 = 1;  CHECK(!bonsai_decode_path_ok(&s), "rejects non-F32 activations");
    s = base(); s.type2 = 1;  CHECK(!bonsai_decode_path_ok(&s), "rejects non-F32 dst");
    s = base(); s.ne20 = 4;   CHECK(!bonsai_decode_path_ok(&s), "rejects 3-D weights");
    s = base(); s.ne30 = 2;   CHECK(!bonsai_decode_path_ok(&s), "rejects 4-D weights");
    s = base(); s.ne11 = 8;   CHECK(!bonsai_decode_path_ok(&s), "rejects batch > 1");
    s = base(); s.ne12 = 2;   CHECK(!bonsai_decode_path_ok(&s), "rejects src1 ne[2] != 1");
    s = base(); s.ne13 = 2;   CHECK(!bonsai_decode_path_ok(&s), "rejects src1 ne[3] != 1");
    s = base(); s.dst_ne1 = 2; CHECK(!bonsai_decode_path_ok(&s), "rejects multi-column dst");
    s = base(); s.n_in = 0;   CHECK(!bonsai_decode_path_ok(&s), "rejects n_in == 0");
    s = base(); s.n_out = 0;  CHECK(!bonsai_decode_path_ok(&s), "rejects n_out == 0");
    s = base(); s.n_in = 5121; s.nb1 = 40 * 34; CHECK(!bonsai_decode_path_ok(&s), "rejects n_in % 128");
    s = base(); s.n_in = 65536; s.nb1 = 65536 / 128 * 34; CHECK(!bonsai_decode_path_ok(&s), "rejects n_in > 32768");
    s = base(); s.nb1 = 4096; CHECK(!bonsai_decode_path_ok(&s), "rejects non-contiguous rows");
    CHECK(BONSAI_MAX_ROW >= 17408, "scratch covers n_ff");
    printf("%d passed, %d failed\n", passes, fails);
    return fails != 0;
}
