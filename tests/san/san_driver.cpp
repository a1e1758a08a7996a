// san_driver.cpp -- the library's host code under AddressSanitizer and
// UndefinedBehaviorSanitizer, on the CPU (no GPU call is made).
//
// Built by tests/san/build.sh from the library sources compiled host-only
// (device code is not compiled, so no kernel exists to launch).  For every
// file named on the command line it runs the GGUF reader the way a loader
// does (GgufReader.open, GgufReader.java:102-183, and the llamafile ZIP paths
// :808-1154): open, info, every tensor's info and raw bytes (bounded), the
// metadata accessors, close.  A call may fail, but only with JH_EFORMAT or
// JH_EIO (JH_EUNSUPPORTED for an unknown tensor type) and a message; any
// other outcome, or a sanitizer report, fails the run.  Then the argument
// checks of host entry points that need no device.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../include/junohip.h"

static int g_bad = 0;

static void expect(bool ok, const char *what, const char *path, int rc) {
    if (!ok) {
        fprintf(stderr, "UNEXPECTED %s on %s: rc=%d (%s)\n", what, path, rc, jh_last_error());
        g_bad++;
    }
}

static bool reader_error(int rc) { return rc == JH_EFORMAT || rc == JH_EIO || rc == JH_EUNSUPPORTED; }

static void read_file(const char *path) {
    jh_gguf *g = nullptr;
    int rc = jh_gguf_open(path, &g);
    if (rc != JH_OK) {
        expect(reader_error(rc) && g == nullptr && strlen(jh_last_error()) > 0, "open result", path, rc);
        return;
    }
    int version = 0;
    int64_t nt = 0, nkv = 0, goff = 0, doff = 0, mend = 0;
    rc = jh_gguf_info(g, &version, &nt, &nkv, &goff, &doff, &mend);
    expect(rc == JH_OK && nt >= 0 && nkv >= 0, "info", path, rc);
    std::vector<unsigned char> buf(1 << 16);
    for (int64_t i = 0; i < nt && i < 4096; i++) {
        const char *name = nullptr;
        int type = 0, nd = 0;
        int64_t dims[8] = {}, ne = 0, off = 0;
        rc = jh_gguf_tensor_info(g, i, &name, &type, &nd, dims, &ne, &off);
        expect(rc == JH_OK && name != nullptr && nd >= 0 && nd <= 8, "tensor_info", path, rc);
        if (rc != JH_OK) continue;
        int64_t idx = -2;
        rc = jh_gguf_tensor_index(g, name, &idx);  // -1 for a name with a NUL inside (not a C string's name)
        expect(rc == JH_OK && idx >= -1 && idx < nt, "tensor_index", path, rc);
        size_t nb = 0;
        rc = jh_gguf_tensor_read(g, i, nullptr, 0, &nb);
        expect(rc == JH_OK || reader_error(rc), "tensor_read (size)", path, rc);
        if (rc == JH_OK && nb <= buf.size()) {
            rc = jh_gguf_tensor_read(g, i, buf.data(), buf.size(), &nb);
            expect(rc == JH_OK || reader_error(rc), "tensor_read", path, rc);
        }
    }
    int64_t idx = 0;
    expect(jh_gguf_tensor_info(g, nt, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == JH_EINVAL,
           "tensor_info past the end", path, -1);
    (void)jh_gguf_tensor_index(g, "no such tensor", &idx);
    const char *keys[] = {"general.architecture", "general.alignment", "llama.context_length", "k_bool", "k_str",
                          "k_arr", "k_f64", "k_i8", "tokenizer.ggml.tokens", ""};
    char s[64];
    for (const char *k : keys) {
        int vt = 0, et = 0, present = 0, bv = 0;
        int64_t cnt = 0, lv = 0;
        double dv = 0;
        size_t len = 0;
        expect(jh_gguf_meta_type(g, k, &vt, &et, &cnt) == JH_OK, "meta_type", path, -1);
        expect(jh_gguf_meta_number(g, k, &present, &lv, &dv) == JH_OK, "meta_number", path, -1);
        expect(jh_gguf_meta_bool(g, k, &present, &bv) == JH_OK, "meta_bool", path, -1);
        expect(jh_gguf_meta_string(g, k, s, sizeof s, &len) == JH_OK, "meta_string", path, -1);
        expect(jh_gguf_meta_string(g, k, s, 1, &len) == JH_OK, "meta_string (cap 1)", path, -1);
    }
    expect(jh_gguf_close(g) == JH_OK, "close", path, -1);
}

// host-side argument checks that return before any device call
static void api_checks() {
    int64_t out = 0;
    for (int t = -3; t < 40; t++) (void)jh_raw_byte_count(t, 256, &out);
    // rawByteCount's formula as the reference writes it (no checks; long arithmetic)
    expect(jh_raw_byte_count(12, -256, &out) == JH_OK && out == -144, "raw_byte_count(negative)", "api", -1);
    expect(jh_raw_byte_count(12, 255, &out) == JH_OK && out == 0, "raw_byte_count(ragged)", "api", -1);
    expect(jh_raw_byte_count(8, INT64_MAX, &out) == JH_OK, "raw_byte_count(huge)", "api", -1);
    expect(jh_raw_byte_count(12, 256, nullptr) == JH_EINVAL, "raw_byte_count(NULL)", "api", -1);
    expect(jh_gguf_open(nullptr, nullptr) == JH_EINVAL, "gguf_open(NULL)", "api", -1);
    expect(jh_gguf_close(nullptr) == JH_OK, "gguf_close(NULL)", "api", -1);
    jh_gguf *g = nullptr;
    const int rc = jh_gguf_open("/nonexistent/dir/model.gguf", &g);
    expect(rc == JH_EIO && g == nullptr, "gguf_open(missing)", "api", rc);
    expect(jh_qmat_free(nullptr) == JH_OK, "qmat_free(NULL)", "api", -1);
    expect(jh_qmatvec_group_dev(9, nullptr, nullptr, nullptr, nullptr) == JH_EINVAL, "group_dev(9)", "api", -1);
}

int main(int argc, char **argv) {
    api_checks();
    for (int i = 1; i < argc; i++) read_file(argv[i]);
    printf("san-driver files %d unexpected %d\n", argc - 1, g_bad);
    return g_bad ? 1 : 0;
}
