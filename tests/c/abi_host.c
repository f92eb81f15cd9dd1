/* Plain C99 consumer of include/zjai_hip.h: the host-side entry points (tiling geometry, region
 * grids, weight readers, bundles, error reporting) called through the C-ABI alone, as a binding
 * written in any language would call them. Built by tests/test_c_abi.py with gcc -std=c99 and
 * AddressSanitizer + UndefinedBehaviorSanitizer; no device is touched.
 *
 * Known answers: the config-5 tiling (src/tools/tiles.rs:127-216 with the encoder's choice for
 * 2x3 independent regions, src/encoder/tiles.rs:294-317: tile 640, overlap 128), the
 * tiles.rs:522-556 region KAT, the regions.rs:155-170 axis KAT, and a 128-byte ZJM1 file
 * assembled by hand from the layout of src/weights/packed.rs:12-21 (one f32 tensor "w" =
 * [1, -2], one integer entry "e" = 5). */

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "zjai_hip.h"

static int failures = 0;

#define CHECK(cond)                                                             \
    do {                                                                        \
        if (!(cond)) {                                                          \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            failures++;                                                         \
        }                                                                       \
    } while (0)

static void test_config5_tiles(void) {
    enum { CAP = 64 };
    zjai_tile t[CAP];
    int32_t n = 0;
    const int32_t h = 2160, w = 3840;
    int32_t i, sizes = 0;
    int32_t seen[8][2];
    unsigned char* cover;
    long long covered = 0, twice = 0;
    CHECK(zjai_synthesis_tiles(h, w, 135, 240, 640, 128, 2, 3, t, CAP, &n) == ZJAI_OK);
    CHECK(n == 24);
    cover = (unsigned char*)calloc((size_t)h * w, 1);
    CHECK(cover != NULL);
    if (!cover) return;
    for (i = 0; i < n; ++i) {
        int32_t j, y, x, known = 0;
        /* A tile's latent window is ceil(image / 16) at image / 16 (latent_extent). */
        CHECK(t[i].latent_w == (t[i].image_w + 15) / 16 && t[i].latent_h == (t[i].image_h + 15) / 16);
        CHECK(t[i].latent_x * 16 == t[i].image_x && t[i].latent_y * 16 == t[i].image_y);
        CHECK(t[i].core_x == t[i].image_x + t[i].core_off_x && t[i].core_y == t[i].image_y + t[i].core_off_y);
        for (j = 0; j < sizes; ++j)
            if (seen[j][0] == t[i].image_w && seen[j][1] == t[i].image_h) known = 1;
        if (!known && sizes < 8) {
            seen[sizes][0] = t[i].image_w;
            seen[sizes][1] = t[i].image_h;
            sizes++;
        }
        for (y = t[i].core_y; y < t[i].core_y + t[i].core_h; ++y)
            for (x = t[i].core_x; x < t[i].core_x + t[i].core_w; ++x) {
                if (y < 0 || y >= h || x < 0 || x >= w) { twice++; continue; }
                if (cover[(size_t)y * w + x]++) twice++;
                else covered++;
            }
    }
    CHECK(sizes == 4); /* 640 x 640, 704 x 704, 768 x 704, 304 x 704 (width x height classes) */
    CHECK(covered == (long long)h * w && twice == 0); /* the cores partition the picture */
    free(cover);
    /* tiles.rs:522-556: two regions split at x = 1024. */
    CHECK(zjai_synthesis_tiles(1400, 2096, 88, 131, 640, 128, 1, 2, t, CAP, &n) == ZJAI_OK);
    CHECK(n == 12);
    CHECK(t[6].latent_x == 76 && t[6].latent_y == 36 && t[6].latent_w == 48 && t[6].latent_h == 48);
    CHECK(t[6].core_x == 1280 && t[6].core_y == 640 && t[6].core_w == 640 && t[6].core_h == 640);
    CHECK(t[6].core_off_x == 64 && t[6].core_off_y == 64);
    /* A capacity that is too small is a limit, not an overflow. */
    CHECK(zjai_synthesis_tiles(2160, 3840, 135, 240, 640, 128, 2, 3, t, 4, &n) == ZJAI_E_LIMIT);
    /* Degenerate tiling: tile not larger than its overlap. */
    CHECK(zjai_synthesis_tiles(1400, 2096, 88, 131, 64, 64, 0, 0, t, CAP, &n) == ZJAI_E_INVALID_ARGUMENT);
}

static void test_region_grid(void) {
    zjai_regions r;
    zjai_area core[16], ext[16];
    int32_t n = 0, i;
    long long area = 0;
    memset(&r, 0, sizeof r);
    r.num_ver = 2;
    r.num_hor = 3;
    r.independent = 1;
    CHECK(zjai_region_grid(2160, 3840, 0, &r, ZJAI_PLANE_LATENT, core, ext, 16, &n) == ZJAI_OK);
    CHECK(n == 6);
    for (i = 0; i < n; ++i) {
        area += (long long)core[i].width * core[i].height;
        CHECK(core[i].x == ext[i].x && core[i].width == ext[i].width); /* independent: not extended */
    }
    CHECK(area == 135LL * 240);
    /* regions.rs:155-170: 3000 rows in 3 regions split at latent rows 64 and 128. */
    r.num_ver = 3;
    r.num_hor = 1;
    CHECK(zjai_region_grid(3000, 100, 0, &r, ZJAI_PLANE_LATENT, core, ext, 16, &n) == ZJAI_OK);
    CHECK(n == 3 && core[0].y == 0 && core[1].y == 64 && core[2].y == 128 && core[2].height == 60);
}

static const unsigned char KNOWN_ZJM1[128] = {
    0x5a, 0x4a, 0x4d, 0x31, 1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0,   /* magic, version, 1, 1 */
    1, 0, 0x77, 1, 1, 2, 0, 0, 0, 0, 0, 0, 0,                     /* "w", F32, rank 1, dim 2 */
    64, 0, 0, 0, 0, 0, 0, 0, 8, 0, 0, 0, 0, 0, 0, 0,              /* offset 64, 8 bytes */
    1, 0, 0x65, 5, 0, 0, 0, 0, 0, 0, 0,                           /* "e" = 5 */
    0, 0, 0, 0, 0, 0, 0, 0,                                       /* pad to 64 */
    0, 0, 0x80, 0x3f, 0, 0, 0, 0xc0};                             /* 1.0, -2.0, pad to 128 */

static void test_checkpoint(void) {
    zjai_checkpoint* ck = NULL;
    int32_t tensors = -1, ints = -1, lists = -1, packed = -1, dtype = -1, rank = -1;
    int64_t shape[ZJAI_MAX_RANK], value = 0;
    char name[32], msg[256];
    float w[2] = {0, 0};
    const char* names[1] = {"w"};
    unsigned char out[256];
    size_t len = 0;
    CHECK(zjai_checkpoint_parse(KNOWN_ZJM1, sizeof KNOWN_ZJM1, &ck) == ZJAI_OK);
    if (!ck) return;
    CHECK(zjai_checkpoint_counts(ck, &tensors, &ints, &lists, &packed) == ZJAI_OK);
    CHECK(tensors == 1 && ints == 1 && lists == 0 && packed == 1);
    CHECK(zjai_checkpoint_tensor_name(ck, 0, name, sizeof name) == ZJAI_OK && strcmp(name, "w") == 0);
    CHECK(zjai_checkpoint_tensor_name(ck, 0, name, 1) == ZJAI_E_LIMIT);
    CHECK(zjai_checkpoint_info(ck, "w", &dtype, &rank, shape) == ZJAI_OK);
    CHECK(dtype == ZJAI_DTYPE_F32 && rank == 1 && shape[0] == 2);
    CHECK(zjai_checkpoint_read_f32(ck, "w", w, 2) == ZJAI_OK && w[0] == 1.0f && w[1] == -2.0f);
    CHECK(zjai_checkpoint_read_f32(ck, "w", w, 3) != ZJAI_OK);
    CHECK(zjai_checkpoint_read_f32(ck, "missing", w, 2) == ZJAI_E_MODEL);
    CHECK(zjai_checkpoint_int_at(ck, 0, name, sizeof name, &value) == ZJAI_OK);
    CHECK(strcmp(name, "e") == 0 && value == 5);
    CHECK(zjai_checkpoint_write_zjm(ck, names, 1, 0, NULL, 0, &len) == ZJAI_OK && len == 128);
    CHECK(zjai_checkpoint_write_zjm(ck, names, 1, 0, out, sizeof out, &len) == ZJAI_OK);
    CHECK(len == 128 && memcmp(out, KNOWN_ZJM1, 128) == 0); /* the writer reproduces the file */
    CHECK(zjai_checkpoint_destroy(ck) == ZJAI_OK);
    /* Truncated and damaged files fail as Error::Model with a message. */
    ck = NULL;
    CHECK(zjai_checkpoint_parse(KNOWN_ZJM1, 40, &ck) == ZJAI_E_MODEL && ck == NULL);
    CHECK(zjai_last_error(NULL, msg, sizeof msg) == ZJAI_OK && msg[0] != 0);
    memcpy(out, KNOWN_ZJM1, 128);
    out[20] = 9; /* rank 9 > ZJAI_MAX_RANK */
    CHECK(zjai_checkpoint_parse(out, 128, &ck) == ZJAI_E_MODEL && ck == NULL);
}

static void test_bundle(void) {
    const char* paths[1] = {"VM_common_int/Y_0.012.pth"};
    const void* files[1] = {KNOWN_ZJM1};
    const size_t sizes[1] = {sizeof KNOWN_ZJM1};
    size_t len = 0, flen = 0;
    unsigned char* buf;
    zjai_bundle* b = NULL;
    int32_t n = 0;
    char path[64];
    const void* data = NULL;
    CHECK(zjai_bundle_write(paths, files, sizes, 1, "notice", 0, NULL, 0, &len) == ZJAI_OK && len > 128);
    buf = (unsigned char*)malloc(len);
    CHECK(buf != NULL);
    if (!buf) return;
    CHECK(zjai_bundle_write(paths, files, sizes, 1, "notice", 0, buf, len, &len) == ZJAI_OK);
    CHECK(zjai_bundle_parse(buf, len, &b) == ZJAI_OK);
    free(buf); /* the bundle holds its own copy */
    if (!b) return;
    CHECK(zjai_bundle_count(b, &n) == ZJAI_OK && n == 1);
    CHECK(zjai_bundle_path(b, 0, path, sizeof path) == ZJAI_OK && strcmp(path, paths[0]) == 0);
    CHECK(zjai_bundle_get(b, paths[0], &data, &flen) == ZJAI_OK);
    CHECK(flen == sizeof KNOWN_ZJM1 && data != NULL && memcmp(data, KNOWN_ZJM1, flen) == 0);
    CHECK(zjai_bundle_get(b, "absent", &data, &flen) != ZJAI_OK);
    CHECK(zjai_bundle_destroy(b) == ZJAI_OK);
}

static void test_null_arguments(void) {
    int32_t n = 0;
    CHECK(zjai_ctx_create(0, 0, NULL) == ZJAI_E_INVALID_ARGUMENT);
    CHECK(zjai_synthesis_tiles(64, 64, 4, 4, 0, 0, 0, 0, NULL, 4, &n) == ZJAI_E_INVALID_ARGUMENT);
    CHECK(zjai_checkpoint_parse(NULL, 10, NULL) == ZJAI_E_INVALID_ARGUMENT);
    CHECK(zjai_ctx_destroy(NULL) == ZJAI_OK);
}

int main(void) {
    test_config5_tiles();
    test_region_grid();
    test_checkpoint();
    test_bundle();
    test_null_arguments();
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("abi_host: all checks passed\n");
    return 0;
}
