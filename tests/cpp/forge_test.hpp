// Shared check macro of the forge:: C++ tests (the reference's tests use the
// same pass/fail counting style).
#pragma once
#include <cmath>
#include <exception>
#include <iostream>

static int g_pass = 0, g_fail = 0;

#define CHECK(name, expr)                                              \
    do {                                                               \
        if (expr) {                                                    \
            g_pass++;                                                  \
            std::cout << "  ok   " << (name) << "\n";                  \
        } else {                                                       \
            g_fail++;                                                  \
            std::cerr << "  FAIL " << (name) << "\n";                  \
        }                                                              \
    } while (0)

static int finish(const char* suite) {
    std::cout << "\n" << suite << ": " << g_pass << " passed, " << g_fail << " failed\n";
    return g_fail ? 1 : 0;
}

// Each test defines run(); library errors (no GPU, bad shapes) end the test
// with status 2 and the library's message.
int run();

int main() {
    try {
        return run();
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 2;
    }
}
