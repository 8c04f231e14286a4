// Test infrastructure only: a main() for the reference's own `inspect` command (GGML-Loader
// src/cmd_inspect.cpp, dispatched as src/main.cpp:14 does), compiled from its source by
// Makefile.ref against this repository's include/ and libggml.so, so that the tests can compare
// bin/ggml-loader inspect with it byte for byte.
int cmd_inspect(int argc, char ** argv);

int main(int argc, char ** argv) {
    return argc < 2 ? 1 : cmd_inspect(argc - 1, argv + 1);
}
