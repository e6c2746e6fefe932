function mlp2_ce_d(loss, lossd, x, xd, lab, w1, w1d, b1, b1d, w2, w2d, b2, b2d, h1, h1d, z, zd, i_b, i_in, i_h, i_out)
    for idx = 1:i_b * i_h
        __icse_0 = idx - 1
        i_s = div(__icse_0, i_h) + 1
        i_j = mod(__icse_0, i_h) + 1
        s1d = b1d[i_j]
        s1 = b1[i_j]
        for i_k = 1:i_in
            __icse_1 = (i_k - 1) * i_h + i_j
            __icse_2 = (i_s - 1) * i_in + i_k
            __cse_3 = x[__icse_2]
            __cse_4 = w1[__icse_1]
            s1d = s1d + (__cse_3 * w1d[__icse_1] + __cse_4 * xd[__icse_2])
            s1 = s1 + __cse_4 * __cse_3
        end
        __cse_5 = tanh(s1)
        __icse_6 = (i_s - 1) * i_h + i_j
        h1d[__icse_6] = (1.0 - __cse_5 ^ 2) * s1d
        h1[__icse_6] = __cse_5
    end
    for idx2 = 1:i_b * i_out
        __icse_7 = idx2 - 1
        i_s2 = div(__icse_7, i_out) + 1
        i_o = mod(__icse_7, i_out) + 1
        s2d = b2d[i_o]
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            __icse_8 = (i_k2 - 1) * i_out + i_o
            __icse_9 = (i_s2 - 1) * i_h + i_k2
            __cse_10 = h1[__icse_9]
            __cse_11 = w2[__icse_8]
            s2d = s2d + (__cse_10 * w2d[__icse_8] + __cse_11 * h1d[__icse_9])
            s2 = s2 + __cse_11 * __cse_10
        end
        __icse_12 = (i_s2 - 1) * i_out + i_o
        zd[__icse_12] = s2d
        z[__icse_12] = s2
    end
    for i_s3 = 1:i_b
        sed = 0.0
        se = 0.0
        for i_o2 = 1:i_out
            __icse_13 = (i_s3 - 1) * i_out + i_o2
            __cse_14 = exp(z[__icse_13])
            sed = sed + __cse_14 * zd[__icse_13]
            se = se + __cse_14
        end
        i_l = lab[i_s3]
        __icse_15 = (i_s3 - 1) * i_out + i_l
        lossd[1] = lossd[1] + ((1.0 / se) * sed + -(zd[__icse_15]))
        loss[1] = loss[1] + (log(se) - z[__icse_15])
    end
    return nothing
end

function mlp2_ce(loss, x, lab, w1, b1, w2, b2, h1, z, i_b, i_in, i_h, i_out)
    # hidden layer: one iteration per (sample, unit); the feature sum is carried (rule 1)
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s1 = b1[i_j]
        for i_k = 1:i_in
            s1 = s1 + w1[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        h1[(i_s - 1) * i_h + i_j] = tanh(s1)
    end
    # output layer: one iteration per (sample, class)
    for idx2 = 1:i_b * i_out
        i_s2 = div(idx2 - 1, i_out) + 1
        i_o = mod(idx2 - 1, i_out) + 1
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            s2 = s2 + w2[(i_k2 - 1) * i_out + i_o] * h1[(i_s2 - 1) * i_h + i_k2]
        end
        z[(i_s2 - 1) * i_out + i_o] = s2
    end
    # softmax cross-entropy of each sample, summed over the batch
    for i_s3 = 1:i_b
        se = 0.0
        for i_o2 = 1:i_out
            se = se + exp(z[(i_s3 - 1) * i_out + i_o2])
        end
        i_l = lab[i_s3]
        loss[1] = loss[1] + (log(se) - z[(i_s3 - 1) * i_out + i_l])
    end
    return nothing
end
