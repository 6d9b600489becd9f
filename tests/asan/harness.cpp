// Sanitizer harness for the host-side model-file readers (test infrastructure): each file named on the command
// line goes through one reader; AddressSanitizer / UndefinedBehaviorSanitizer report any invalid access.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include "eif_hip.h"
#include "eif_hip_gguf.h"
#include "eif_hip_qwen35.h"
// the GPU side of the library is not linked: these stand-ins are never reached by the parsers under test
extern "C" {
int eif_hip_bitnet_create(eif_hip_bitnet **, const eif_hip_bitnet_config *) { return -2; }
int eif_hip_bitnet_set_layer(eif_hip_bitnet *, int, const eif_hip_bitnet_layer *) { return -2; }
int eif_hip_bitnet_set_globals(eif_hip_bitnet *, const eif_hip_bitnet_globals *) { return -2; }
void eif_hip_bitnet_destroy(eif_hip_bitnet *) {}
int eif_hip_qweight_create(eif_hip_qweight **, int, int, int, int, const void *, const float *, int, void *) { return -2; }
void eif_hip_qweight_destroy(eif_hip_qweight *) {}
int eif_hip_qlinear_prep(const eif_hip_qweight *, const eif_hip_prep_spec *, const float *, float *, int, int, void *) { return -2; }
int eif_hadamard_block_size(int n) { int b = 1; while (b < 1024 && n % (2 * b) == 0) b *= 2; return b; }
int eif_bitnet_group_size(int n, int mx) { for (int g = mx / 32 * 32; g >= 32; g -= 32) if (n % g == 0) return g; return 0; }
float eif_hip_wht_norm(int) { return 1.0f; }
}
static std::vector<unsigned char> slurp(const char *p) {
    std::vector<unsigned char> b; FILE *f = fopen(p, "rb"); if (!f) return b;
    fseek(f, 0, SEEK_END); long n = ftell(f); fseek(f, 0, SEEK_SET); b.resize(n > 0 ? n : 0);
    if (n > 0 && fread(b.data(), 1, n, f) != (size_t)n) b.clear(); fclose(f); return b;
}
int main(int argc, char **argv) {
    int ok[3] = {0, 0, 0}, n[3] = {0, 0, 0};
    for (int i = 2; i < argc; ++i) {
        const char *p = argv[i];
        if (!strcmp(argv[1], "bitnet")) {
            eif_gguf_bitnet *m = nullptr;
            ++n[0];
            if (eif_gguf_bitnet_open(&m, p) == 0) { ++ok[0]; eif_gguf_bitnet_close(m); }
        } else if (!strcmp(argv[1], "svlm")) {
            eif_hip_bitnet *m = nullptr;
            ++n[0];
            if (eif_hip_bitnet_load_svlm(&m, p, 0) == -2) ++ok[0];   // reached the decoder's create
        } else if (!strcmp(argv[1], "q35gguf")) {
            auto b = slurp(p); void *img = nullptr; size_t sz = 0; ++n[1];
            if (eif_qwen35_gguf_image(b.data(), b.size(), &img, &sz) == 0) { ++ok[1]; eif_qwen35_image_free(img); }
        } else {
            auto b = slurp(p); eif_qwen35_layout lay; ++n[2];
            if (eif_qwen35_parse(b.data(), b.size(), &lay) == 0) ++ok[2];
        }
    }
    printf("%s: %d/%d/%d ok of %d/%d/%d\n", argv[1], ok[0], ok[1], ok[2], n[0], n[1], n[2]);
    return 0;
}
