/* knx_fuzz.c — loader fuzz harness (run by tests/test_fuzz.py, built with AddressSanitizer and UBSan over the host
 * runtime sources).  Loads every file named on the command line and frees the accepted ones; with --forward it also
 * runs a 3-sample forward, then the same with a 1-byte workspace limit (one sample per chunk), as the reference's
 * harness does (reference test/knx_fuzz.c:6-24).  Prints "loaded N / M". */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernix_model.h"

int main(int argc, char** argv)
{
    int first = 1, forward = 0, loaded = 0;
    if (argc > 1 && strcmp(argv[1], "--forward") == 0) { forward = 1; first = 2; }
    for (int i = first; i < argc; i++) {
        kernix_model* m = kernix_model_load(argv[i]);
        if (m == NULL) continue;
        loaded++;
        const size_t rows = 3 * (size_t)m->seq_len, n = rows * (size_t)m->in_dim;
        if (forward && n <= ((size_t)1 << 24)) {
            float* data = malloc(sizeof(float) * (n ? n : 1));
            if (data != NULL) {
                for (size_t k = 0; k < n; k++) data[k] = (float)((k * 2654435761u) % 7) - 3.0f;
                float_tensor x = { (int)rows, m->in_dim, data };
                kernix_model_forward(m, &x);
                kernix_model_set_workspace_limit(m, 1);
                kernix_model_forward(m, &x);
                free(data);
            }
        }
        kernix_model_free(m);
    }
    printf("loaded %d / %d\n", loaded, argc - first);
    return 0;
}
