"""Torch-free input generators shared by the CPU and GPU tests."""
import numpy as np


def special_input(batch, classes, anchors, frame):
    # CpuPtEndToEndTests.cs:58-86.
    x = np.zeros((batch, classes + 4, anchors), np.float32)
    for b in range(batch):
        for c in range(4):
            for a in range(anchors):
                x[b, c, a] = b * 10000 + c * 1000 + a + frame * 100000
        for c in range(classes):
            for a in range(anchors):
                score = np.float32(((a * 7 + c * 3 + frame) % 17 - 8) / np.float32(10))
                k = (a + c * 3 + frame) % 13
                if k == 0:
                    score = np.array([0x7fc00001 + a + c], np.uint32).view(np.float32)[0]
                elif k == 1:
                    score = np.float32(np.inf)
                elif k == 2:
                    score = np.float32(-np.inf)
                elif k == 3:
                    score = np.float32(0)
                elif k == 4:
                    score = np.array([0x80000000], np.uint32).view(np.float32)[0]
                elif k == 5:
                    score = np.array([1], np.uint32).view(np.float32)[0]
                elif k == 6:
                    score = np.array([0x80000001], np.uint32).view(np.float32)[0]
                if frame == 3:
                    score = np.float32(a % 7 * np.float32(0.1)) if c == 0 else np.float32(0.25)
                x[b, 4 + c, a] = score
    return x
